// kernels.hip — gfx950 kernels of the Qwen3 decode step (and the op-level
// entries). Each kernel reproduces the reference AVX2 arithmetic exactly;
// the reference function it replaces is cited at each kernel.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"
#include "rlh_device.h"

namespace rlh {

// ---------------------------------------------------------------------------
// Embedding gather: x[t][i] = dequant_row(token_embd, tok[t])[i]
// (model.rs:612-614, 414-418 -> tensor.rs:59-62 -> quant.rs:191-385).
// grid (ceil(E/256), n_tokens), block 256.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_embed(DevMat w, const uint32_t* tok, float* x) {
  uint32_t i = blockIdx.x * 256 + threadIdx.x;
  uint32_t t = blockIdx.y;
  if (i >= w.cols) return;
  uint32_t row = tok[t];
  if (row >= w.rows) row = 0;  // ids are validated on the host; never read out of bounds
  x[(size_t)t * w.cols + i] = dq_elem(w, row, i);
}

// ---------------------------------------------------------------------------
// rmsnorm (simd.rs:282-326) fused with quantize_q8 (simd.rs:116-203) of the
// result: xb = (x*s)*w, s = 1/sqrt(ss/n + eps); Q8 blocks of xb.
// One 256-thread block per token (grid.x = n_tokens). n % 32 == 0.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_rmsnorm_q8(const float* x, const float* w, int n, float eps, Q8Out out,
                                                    float* xb) {
  __shared__ float s_scale;
  __shared__ __attribute__((aligned(16))) float xs_generic[kMaxEmbd];
  RLH_LDS float* xs = (RLH_LDS float*)xs_generic;
  constexpr int kV = kMaxEmbd / 4 / 256;  // float4 of the row per thread
  const float* xt = x + (size_t)blockIdx.x * n;
  const int n4 = n / 4;
  // Every global load is issued up front (registers), then the row is staged
  // in LDS for the 32 sequential FMA chains of the sum of squares.
  float4 xr[kV], wr[kV];
#pragma unroll
  for (int k = 0; k < kV; k++) {
    const int i = threadIdx.x + 256 * k;
    if (i < n4) {
      xr[k] = ld_gf4(xt + 4 * i);
      wr[k] = ld_gf4(w + 4 * i);
    }
  }
#pragma unroll
  for (int k = 0; k < kV; k++) {
    const int i = threadIdx.x + 256 * k;
    if (i < n4) {
      xs[4 * i] = xr[k].x;
      xs[4 * i + 1] = xr[k].y;
      xs[4 * i + 2] = xr[k].z;
      xs[4 * i + 3] = xr[k].w;
    }
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    float ss = rms_sumsq_lds(xs, n);
    if (threadIdx.x == 0) s_scale = 1.0f / sqrtf(ss / (float)n + eps);
  }
  __syncthreads();
  const float s = s_scale;
  const uint32_t nb = (uint32_t)n / 32;
  Q8Out o{out.qs + (size_t)blockIdx.x * n, out.d + (size_t)blockIdx.x * nb, out.s + (size_t)blockIdx.x * nb,
          out.s16 + (size_t)blockIdx.x * nb * 2};
  // xb = (x * s) * w; 8 consecutive threads hold one Q8 block (4 values each).
#pragma unroll
  for (int k = 0; k < kV; k++) {
    const int i = threadIdx.x + 256 * k;
    if (i < n4) {  // n4 is a multiple of 8: whole 8-lane groups
      const float v0 = (xr[k].x * s) * wr[k].x, v1 = (xr[k].y * s) * wr[k].y;
      const float v2 = (xr[k].z * s) * wr[k].z, v3 = (xr[k].w * s) * wr[k].w;
      if (xb) {
        float* xo = xb + (size_t)blockIdx.x * n + 4 * i;
        xo[0] = v0;
        xo[1] = v1;
        xo[2] = v2;
        xo[3] = v3;
      }
      q8_quant_block8x4(v0, v1, v2, v3, o, (uint32_t)i / 8);
    }
  }
}

// Standalone quantize_q8 (op-level entry): grid covers n/32 blocks, 8 per block.
__global__ void __launch_bounds__(256) k_quantize_q8(const float* x, uint32_t n, Q8Out out) {
  uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (blockIdx.x * 256 + (threadIdx.x & ~31u) >= n) return;  // whole 32-lane halves
  q8_quant_block32(x[i], out, i / 32);
}

// Exact integer partial dots for the op-level parity entry (one thread per
// (row, output value)).
__global__ void __launch_bounds__(256) k_block_dots(DevMat w, const int8_t* a, int32_t* out, uint32_t per_row) {
  size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)w.rows * per_row) return;
  uint32_t row = (uint32_t)(idx / per_row), k = (uint32_t)(idx % per_row);
  int s = 0;
  switch (w.ty) {
    case RLH_TYPE_Q4_K: {  // k = 32-block index: bi*8 + 2g + hi
      const uint32_t bi = k >> 3, g = (k >> 1) & 3, hi = k & 1;
      for (uint32_t l = 0; l < 32; l++)
        s += (int)((item_u8(w, row, bi, 16 + 32 * g + l) >> (4 * hi)) & 0xF) * a[(size_t)k * 32 + l];
      break;
    }
    case RLH_TYPE_Q6_K: {  // k = 16-half index: (bi*8 + half*4 + c)*2 + sub
      const uint32_t blk = k >> 1, sub = k & 1, bi = blk >> 3, half = (blk >> 2) & 1, c = blk & 3;
      for (uint32_t l = 0; l < 16; l++) {
        const uint32_t qlb = item_u8(w, row, bi, half * 64 + (c & 1) * 32 + sub * 16 + l);
        const uint32_t qhb = item_u8(w, row, bi, 128 + half * 32 + sub * 16 + l);
        const uint32_t nib = c < 2 ? (qlb & 0xF) : (qlb >> 4);
        const uint32_t uu = nib | (((qhb >> (2 * c)) & 3) << 4);
        s += (int)uu * a[(size_t)blk * 32 + sub * 16 + l];
      }
      break;
    }
    case RLH_TYPE_Q8_0: {
      const uint32_t j = k >> 3, kk = k & 7;
      for (uint32_t l = 0; l < 32; l++) s += (int)(int8_t)item_u8(w, row, j, kk * 32 + l) * a[(size_t)k * 32 + l];
      break;
    }
    case RLH_TYPE_Q4_0: {
      const uint32_t j = k >> 3, kk = k & 7;
      for (uint32_t l = 0; l < 16; l++) {
        const uint32_t q = item_u8(w, row, j, kk * 16 + l);
        s += (int)(q & 0xF) * a[(size_t)k * 32 + l];
        s += (int)(q >> 4) * a[(size_t)k * 32 + 16 + l];
      }
      break;
    }
    default:
      break;
  }
  out[idx] = s;
}

// Dequantise rows [0, rows) of a matrix into out (row-major f32).
__global__ void __launch_bounds__(256) k_dequant(DevMat w, float* out) {
  size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)w.rows * w.cols) return;
  out[idx] = dq_elem(w, (uint32_t)(idx / w.cols), (uint32_t)(idx % w.cols));
}

// ---------------------------------------------------------------------------
// Per head: (+bias), QK-norm (rmsnorm_head, ops.rs:365-390 -> simd.rs:282-326
// in place), NeoX RoPE (ops.rs:426-446) from the host-built glibc cos/sin
// table, and the K/V write at pos (model.rs:642-656, 466-506).
// Four (head, token) items per block of 256 threads, one per wave (item
// i = token * (H + KVH) + head, q heads first); every wave reaches the
// block's barriers, a wave past the last item works on item 0 and stores
// nothing. q/k/v are token-major [n][dim]; pos of token t is pos0[0] + t.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_qk_norm_rope_kv(float* q, float* k, const float* v, const float* bq,
                                                        const float* bk, const float* bv, const float* qn,
                                                        const float* kn, const float* rope_cs, const uint32_t* pos0,
                                                        float* kcache, float* vcache, int H, int KVH, float eps,
                                                        uint32_t n_items) {
  constexpr int hd = 128;
  __shared__ float hbuf_w[4][hd];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t item = blockIdx.x * 4 + wave;
  const bool live = item < n_items;
  const uint32_t it = live ? item : 0u;
  float* hbuf = hbuf_w[wave];
  int head = (int)(it % (uint32_t)(H + KVH));
  int t = (int)(it / (uint32_t)(H + KVH));
  uint32_t pos = pos0[0] + (uint32_t)t;
  const int qd = H * hd, kvd = KVH * hd;
  bool is_q = head < H;
  int h = is_q ? head : head - H;
  float* src = is_q ? q + (size_t)t * qd + h * hd : k + (size_t)t * kvd + h * hd;
  const float* bias = is_q ? bq : bk;
  const float* nw = is_q ? qn : kn;
  // every global read of the lane first (elements lane and lane + 64: the
  // row, its bias and norm weights, the RoPE pair's cos and sin), so that
  // they are in flight together
  const float x0r = src[lane], x1r = src[lane + 64];
  const float b0 = bias ? bias[h * hd + lane] : 0.0f, b1 = bias ? bias[h * hd + lane + 64] : 0.0f;
  const float w0 = nw ? nw[lane] : 0.0f, w1 = nw ? nw[lane + 64] : 0.0f;
  const float c = rope_cs[(size_t)pos * hd + 2 * lane];
  const float sn = rope_cs[(size_t)pos * hd + 2 * lane + 1];
  hbuf[lane] = bias ? x0r + b0 : x0r;
  hbuf[lane + 64] = bias ? x1r + b1 : x1r;
  __syncthreads();
  if (nw) {
    float ss = rms_sumsq_wave(hbuf, hd);
    float s = 1.0f / sqrtf(ss / (float)hd + eps);
    __syncthreads();
    hbuf[lane] = hbuf[lane] * s * w0;
    hbuf[lane + 64] = hbuf[lane + 64] * s * w1;
    __syncthreads();
  }
  // RoPE pairs (i, i+64): lane i < 64 handles pair i.
  {
    int i = lane;
    float x0 = hbuf[i], x1 = hbuf[i + 64];
    float y0 = x0 * c - x1 * sn;
    float y1 = x0 * sn + x1 * c;
    if (!live) {
    } else if (is_q) {
      src[i] = y0;
      src[i + 64] = y1;
    } else {
      float* kd = kcache + (size_t)pos * kvd + h * hd;
      kd[i] = y0;
      kd[i + 64] = y1;
      if (v) {  // null: the v product wrote its rows into the cache itself
        const float* vs = v + (size_t)t * kvd + h * hd;
        float* vd = vcache + (size_t)pos * kvd + h * hd;
        for (int j = lane; j < hd; j += 64) {
          float x = vs[j];
          if (bv) x = x + bv[h * hd + j];
          vd[j] = x;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// SwiGLU + Q8: h = silu(g) * u, silu(x) = x / (1 + expf(-x)) (ops.rs:393-395,
// model.rs:722-724, 565-567), then quantize_q8 of h (ffn_down input).
// grid covers n_total = n_tokens * F elements, 256 per block.
// ---------------------------------------------------------------------------
// Four consecutive values per thread (16-byte loads), eight threads per Q8
// block of 32; the expf table in LDS. n_total is a multiple of 32, so a
// block of 32 values never straddles the end.
__global__ void __launch_bounds__(256) k_swiglu_q8(const float* g, const float* u, uint32_t n_total, Q8Out out,
                                                   float* h_out) {
  __shared__ uint64_t tab_g[32];
  lu64* tab = (lu64*)tab_g;
  exp_tab_to_lds(tab);
  __syncthreads();
  const uint32_t i4 = blockIdx.x * 256 + threadIdx.x;  // float4 index
  if (blockIdx.x * 256 + (threadIdx.x & ~7u) >= n_total / 4) return;
  const float4 x = ((const float4*)g)[i4], uu = ((const float4*)u)[i4];
  // ops.rs:393-395 per value: silu(x) = x / (1 + exp(-x)), times up
  const float h0 = (x.x / (1.0f + expf_glibc_t(-x.x, tab))) * uu.x;
  const float h1 = (x.y / (1.0f + expf_glibc_t(-x.y, tab))) * uu.y;
  const float h2 = (x.z / (1.0f + expf_glibc_t(-x.z, tab))) * uu.z;
  const float h3 = (x.w / (1.0f + expf_glibc_t(-x.w, tab))) * uu.w;
  if (h_out) ((float4*)h_out)[i4] = float4{h0, h1, h2, h3};
  q8_quant_block8x4(h0, h1, h2, h3, out, i4 / 8);
}

// ---------------------------------------------------------------------------
// Argmax with main.rs:453-463 semantics: start at -inf, strict '>' so the
// lowest index among equal maxima wins and NaN never wins.
// Stage 1: per block (value, index); stage 2: one block over the partials,
// writes the token and advances the decode step state.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void argmax_merge(float& bv, uint32_t& bi, float v, uint32_t i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

__global__ void __launch_bounds__(256) k_argmax_partial(const float* x, uint32_t n, float* pv, uint32_t* pi) {
  __shared__ float sv[256];
  __shared__ uint32_t si[256];
  float bv = -__int_as_float(0x7f800000);
  uint32_t bi = 0xffffffffu;
  // 64-bit index: with n near 2^32 a 32-bit i += stride would wrap below n
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256)
    argmax_merge(bv, bi, x[i], (uint32_t)i);
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if ((int)threadIdx.x < st) {
      float v = sv[threadIdx.x + st];
      uint32_t i = si[threadIdx.x + st];
      float b = sv[threadIdx.x];
      uint32_t j = si[threadIdx.x];
      argmax_merge(b, j, v, i);
      sv[threadIdx.x] = b;
      si[threadIdx.x] = j;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    pv[blockIdx.x] = sv[0];
    pi[blockIdx.x] = si[0];
  }
}

// step: when non-null, greedy-loop state: tok_out <- argmax, pos += 1,
// hist[++step] <- argmax. 1024 threads; every thread first issues the loads
// of its partials (up to 16 in flight), then merges them.
__global__ void __launch_bounds__(1024) k_argmax_final(const float* pv, const uint32_t* pi, uint32_t np,
                                                       uint32_t* tok_out, uint32_t* pos, uint32_t* step,
                                                       uint32_t* hist) {
  __shared__ float sv[16];
  __shared__ uint32_t si[16];
  float bv = -__int_as_float(0x7f800000);
  uint32_t bi = 0xffffffffu;
  for (uint32_t i0 = threadIdx.x; i0 < np; i0 += 1024 * 16) {
    float v[16];
    uint32_t ix[16];
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const uint32_t i = i0 + 1024u * k;
      v[k] = i < np ? pv[i] : -__int_as_float(0x7f800000);
      ix[k] = i < np ? pi[i] : 0xffffffffu;
    }
#pragma unroll
    for (int k = 0; k < 16; k++) argmax_merge(bv, bi, v[k], ix[k]);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(bv, m);
    const uint32_t oi = __shfl_xor(bi, m);
    argmax_merge(bv, bi, ov, oi);
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = bv;
    si[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sv[0];
    uint32_t j = si[0];
    for (int k = 1; k < 16; k++) argmax_merge(b, j, sv[k], si[k]);
    // main.rs argmax keeps index 0 unless a value exceeds -inf (all values
    // NaN or -inf -> 0); the merge above takes the first of equal maxima
    const uint32_t best = (j == 0xffffffffu || !(b > -__int_as_float(0x7f800000))) ? 0u : j;
    tok_out[0] = best;
    if (step) {
      const uint32_t s = step[0] + 1;
      hist[s] = best;
      step[0] = s;
      pos[0] = pos[0] + 1;
    }
  }
}

// ---------------------------------------------------------------------------
// Launch wrappers
// ---------------------------------------------------------------------------
static inline Q8Out q8out(const Q8Buf& b) { return Q8Out{b.qs, b.d, b.s, b.s16}; }

void launch_embed(hipStream_t st, const DevMat& w, const uint32_t* tok, uint32_t n_tok, float* x) {
  dim3 grid((w.cols + 255) / 256, n_tok);
  hipLaunchKernelGGL(k_embed, grid, dim3(256), 0, st, w, tok, x);
}

void launch_rmsnorm_q8(hipStream_t st, const float* x, const float* w, uint32_t n, uint32_t n_tok, float eps,
                       const Q8Buf& out, float* xb) {
  hipLaunchKernelGGL(k_rmsnorm_q8, dim3(n_tok), dim3(256), 0, st, x, w, (int)n, eps, q8out(out), xb);
}

void launch_quantize_q8(hipStream_t st, const float* x, uint32_t n, const Q8Buf& out) {
  hipLaunchKernelGGL(k_quantize_q8, dim3((n + 255) / 256), dim3(256), 0, st, x, n, q8out(out));
}

bool matvec_supported(uint32_t ty) {
  return ty == RLH_TYPE_Q4_K || ty == RLH_TYPE_Q6_K || ty == RLH_TYPE_Q8_0 || ty == RLH_TYPE_Q4_0 ||
         ty == RLH_TYPE_Q5_K || ty == RLH_TYPE_Q4_1 || ty == RLH_TYPE_Q5_0 || ty == RLH_TYPE_Q5_1 ||
         ty == RLH_TYPE_F16 || ty == RLH_TYPE_F32 || ty == RLH_TYPE_BF16;
}

void launch_block_dots(hipStream_t st, const DevMat& w, const int8_t* a, int32_t* out, uint32_t per_row) {
  size_t n = (size_t)w.rows * per_row;
  hipLaunchKernelGGL(k_block_dots, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w, a, out, per_row);
}

void launch_dequant(hipStream_t st, const DevMat& w, float* out) {
  size_t n = (size_t)w.rows * w.cols;
  hipLaunchKernelGGL(k_dequant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w, out);
}

void launch_qk_norm_rope_kv(hipStream_t st, float* q, float* k, const float* v, const float* bq, const float* bk,
                            const float* bv, const float* qn, const float* kn, const float* rope_cs,
                            const uint32_t* pos0, float* kcache, float* vcache, int H, int KVH, uint32_t n_tok,
                            float eps) {
  const uint32_t n_items = (uint32_t)(H + KVH) * n_tok;
  hipLaunchKernelGGL(k_qk_norm_rope_kv, dim3((n_items + 3) / 4), dim3(256), 0, st, q, k, v, bq, bk, bv, qn, kn,
                     rope_cs, pos0, kcache, vcache, H, KVH, eps, n_items);
}

void launch_swiglu_q8(hipStream_t st, const float* g, const float* u, uint32_t n_total, const Q8Buf& out,
                      float* h_out) {
  hipLaunchKernelGGL(k_swiglu_q8, dim3((n_total / 4 + 255) / 256), dim3(256), 0, st, g, u, n_total, q8out(out), h_out);
}

void launch_argmax_final(hipStream_t st, const float* pv, const uint32_t* pi, uint32_t nparts, uint32_t* tok_out,
                         uint32_t* pos, uint32_t* step, uint32_t* hist) {
  hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(1024), 0, st, pv, pi, nparts, tok_out, pos, step, hist);
}

void launch_argmax(hipStream_t st, const float* x, uint32_t n, float* pv, uint32_t* pi, uint32_t nparts,
                   uint32_t* tok_out, uint32_t* pos, uint32_t* step, uint32_t* hist) {
  hipLaunchKernelGGL(k_argmax_partial, dim3(nparts), dim3(256), 0, st, x, n, pv, pi);
  hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(1024), 0, st, pv, pi, nparts, tok_out, pos, step, hist);
}

}  // namespace rlh

