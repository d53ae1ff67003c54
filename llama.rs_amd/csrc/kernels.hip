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
  const float* xt = x + (size_t)blockIdx.x * n;
  if (threadIdx.x < 64) {
    float ss = rms_sumsq_wave(xt, n);
    if (threadIdx.x == 0) s_scale = 1.0f / sqrtf(ss / (float)n + eps);
  }
  __syncthreads();
  float s = s_scale;
  uint32_t nb = (uint32_t)n / 32;
  Q8Out o{out.qs + (size_t)blockIdx.x * n, out.d + (size_t)blockIdx.x * nb, out.s + (size_t)blockIdx.x * nb,
          out.s16 + (size_t)blockIdx.x * nb * 2};
  // 8 blocks of 32 per pass (two per wave).
  for (uint32_t base = 0; base < (uint32_t)n; base += 256) {
    uint32_t i = base + threadIdx.x;
    // Waves whose 32-lane halves are past the end skip the pass as a whole half.
    if (base + (threadIdx.x & ~31u) < (uint32_t)n) {
      float v = (xt[i] * s) * w[i];
      if (xb) xb[(size_t)blockIdx.x * n + i] = v;
      q8_quant_block32(v, o, i / 32);
    }
  }
}

// Standalone quantize_q8 (op-level entry): grid covers n/32 blocks, 8 per block.
__global__ void __launch_bounds__(256) k_quantize_q8(const float* x, uint32_t n, Q8Out out) {
  uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (blockIdx.x * 256 + (threadIdx.x & ~31u) >= n) return;  // whole 32-lane halves
  q8_quant_block32(x[i], out, i / 32);
}

// ---------------------------------------------------------------------------
// Decode matvec y = W x (ops.rs:67-141, integer path), exact in the reference
// order: each row's f32 total is the sequential sum, in index order, of the
// per-group terms of dot_q4k_q8_avx2 (simd.rs:581), dot_q6k_q8_avx2
// (simd.rs:663), dot_q80_q8_avx2 (simd.rs:891) or dot_q40_q8_avx2
// (simd.rs:863). Threads compute terms (coalesced over the row's blocks),
// stage them in LDS, and lane r of the block chains row r's terms in order.
// ---------------------------------------------------------------------------
struct Q8In {
  const int8_t* qs;
  const float* d;
  const int32_t* s;
  const int32_t* s16;
};

template <uint32_t TY>
struct Unit;

// Q4_K: unit = group g of super-block bi -> 1 term (64 weights).
template <>
struct Unit<RLH_TYPE_Q4_K> {
  static constexpr int kTerms = 1;
  __device__ static uint32_t units(uint32_t cols) { return cols / 64; }
  __device__ static void run(const DevMat& w, const Q8In& act, uint32_t row, uint32_t u, float* t) {
    uint32_t bi = u >> 2, g = u & 3;
    const uint8_t* sb = w.a + (size_t)row * w.row_bytes + (size_t)bi * 144;
    uint4 hdr = *(const uint4*)sb;
    uint4 q0 = *(const uint4*)(sb + 16 + 32 * g);
    uint4 q1 = *(const uint4*)(sb + 32 + 32 * g);
    uint32_t ab = bi * 8 + 2 * g;
    const uint4* ap = (const uint4*)(act.qs + (size_t)ab * 32);
    uint4 a0 = ap[0], a1 = ap[1], b0 = ap[2], b1 = ap[3];
    const uint32_t m = 0x0F0F0F0Fu;
    int i1 = 0, i2 = 0;
    i1 = sdot4(q0.x & m, a0.x, i1); i1 = sdot4(q0.y & m, a0.y, i1);
    i1 = sdot4(q0.z & m, a0.z, i1); i1 = sdot4(q0.w & m, a0.w, i1);
    i1 = sdot4(q1.x & m, a1.x, i1); i1 = sdot4(q1.y & m, a1.y, i1);
    i1 = sdot4(q1.z & m, a1.z, i1); i1 = sdot4(q1.w & m, a1.w, i1);
    i2 = sdot4((q0.x >> 4) & m, b0.x, i2); i2 = sdot4((q0.y >> 4) & m, b0.y, i2);
    i2 = sdot4((q0.z >> 4) & m, b0.z, i2); i2 = sdot4((q0.w >> 4) & m, b0.w, i2);
    i2 = sdot4((q1.x >> 4) & m, b1.x, i2); i2 = sdot4((q1.y >> 4) & m, b1.y, i2);
    i2 = sdot4((q1.z >> 4) & m, b1.z, i2); i2 = sdot4((q1.w >> 4) & m, b1.w, i2);
    float d = f16_to_f32(hdr.x & 0xffff);
    float dmin = f16_to_f32(hdr.x >> 16);
    uint8_t sc12[12];
    *(uint32_t*)(sc12) = hdr.y;
    *(uint32_t*)(sc12 + 4) = hdr.z;
    *(uint32_t*)(sc12 + 8) = hdr.w;
    uint32_t sc1, m1, sc2, m2;
    scale_min_k4((int)(2 * g), sc12, sc1, m1);
    scale_min_k4((int)(2 * g + 1), sc12, sc2, m2);
    float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
    float d2 = d * (float)sc2, mm2 = dmin * (float)m2;
    float sa = (float)act.s[ab], sb2 = (float)act.s[ab + 1];
    float da = act.d[ab], db = act.d[ab + 1];
    t[0] = da * (d1 * (float)i1 - mm1 * sa) + db * (d2 * (float)i2 - mm2 * sb2);
  }
};

// Q6_K: unit = (bi, half, sub) -> 4 terms c = 0..3 (16 weights each), in the
// reference's loop order half { sub { c } } (simd.rs:617-665).
template <>
struct Unit<RLH_TYPE_Q6_K> {
  static constexpr int kTerms = 4;
  __device__ static uint32_t units(uint32_t cols) { return cols / 64; }
  __device__ static void run(const DevMat& w, const Q8In& act, uint32_t row, uint32_t u, float* t) {
    uint32_t nsb = w.cols >> 8;
    uint32_t bi = u >> 2, half = (u >> 1) & 1, sub = u & 1;
    size_t sbi = (size_t)row * nsb + bi;
    const uint8_t* ql = w.a + sbi * 128 + half * 64 + sub * 16;
    uint4 ql0 = *(const uint4*)ql;
    uint4 ql1 = *(const uint4*)(ql + 32);
    uint4 qh = *(const uint4*)(w.b + sbi * 64 + half * 32 + sub * 16);
    const int8_t* sc = (const int8_t*)(w.c + sbi * 16 + half * 8 + sub);
    const uint8_t* dp = w.d + sbi * 2;
    float d = f16_to_f32(dp[0] | (dp[1] << 8));
    const uint32_t m4 = 0x0F0F0F0Fu, m2 = 0x03030303u;
    uint32_t l0[4] = {ql0.x, ql0.y, ql0.z, ql0.w};
    uint32_t l1[4] = {ql1.x, ql1.y, ql1.z, ql1.w};
    uint32_t h[4] = {qh.x, qh.y, qh.z, qh.w};
    uint32_t ab = bi * 8 + half * 4;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const uint4 a = *(const uint4*)(act.qs + (size_t)(ab + c) * 32 + sub * 16);
      uint32_t av[4] = {a.x, a.y, a.z, a.w};
      int ss = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint32_t lo = (c & 1) ? l1[k] : l0[k];
        uint32_t nib = (c < 2) ? (lo & m4) : ((lo >> 4) & m4);
        uint32_t uu = nib | (((h[k] >> (2 * c)) & m2) << 4);
        ss = sdot4(uu, av[k], ss);
      }
      float scf = (float)sc[2 * c];
      float sa = (float)act.s16[(size_t)(ab + c) * 2 + sub];
      float da = act.d[ab + c];
      t[c] = d * scf * ((float)ss - 32.0f * sa) * da;
    }
  }
};

// Q8_0: unit = one 32-block -> 1 term (simd.rs:874-894).
template <>
struct Unit<RLH_TYPE_Q8_0> {
  static constexpr int kTerms = 1;
  __device__ static uint32_t units(uint32_t cols) { return cols / 32; }
  __device__ static void run(const DevMat& w, const Q8In& act, uint32_t row, uint32_t u, float* t) {
    uint32_t nb = w.cols >> 5;
    size_t b = (size_t)row * nb + u;
    const uint4* qp = (const uint4*)(w.a + b * 32);
    uint4 q0 = qp[0], q1 = qp[1];
    const uint4* ap = (const uint4*)(act.qs + (size_t)u * 32);
    uint4 a0 = ap[0], a1 = ap[1];
    int i = 0;
    i = sdot4(q0.x, a0.x, i); i = sdot4(q0.y, a0.y, i); i = sdot4(q0.z, a0.z, i); i = sdot4(q0.w, a0.w, i);
    i = sdot4(q1.x, a1.x, i); i = sdot4(q1.y, a1.y, i); i = sdot4(q1.z, a1.z, i); i = sdot4(q1.w, a1.w, i);
    float d = f16_to_f32(w.b[2 * b] | (w.b[2 * b + 1] << 8));
    t[0] = d * (float)i * act.d[u];
  }
};

// Q4_0: unit = one 32-block -> 1 term (simd.rs:844-866).
template <>
struct Unit<RLH_TYPE_Q4_0> {
  static constexpr int kTerms = 1;
  __device__ static uint32_t units(uint32_t cols) { return cols / 32; }
  __device__ static void run(const DevMat& w, const Q8In& act, uint32_t row, uint32_t u, float* t) {
    uint32_t nb = w.cols >> 5;
    size_t b = (size_t)row * nb + u;
    uint4 q = *(const uint4*)(w.a + b * 16);
    const uint4* ap = (const uint4*)(act.qs + (size_t)u * 32);
    uint4 a0 = ap[0], a1 = ap[1];
    const uint32_t m = 0x0F0F0F0Fu;
    int i0 = 0, i1 = 0;
    i0 = sdot4(q.x & m, a0.x, i0); i0 = sdot4(q.y & m, a0.y, i0);
    i0 = sdot4(q.z & m, a0.z, i0); i0 = sdot4(q.w & m, a0.w, i0);
    i1 = sdot4((q.x >> 4) & m, a1.x, i1); i1 = sdot4((q.y >> 4) & m, a1.y, i1);
    i1 = sdot4((q.z >> 4) & m, a1.z, i1); i1 = sdot4((q.w >> 4) & m, a1.w, i1);
    float d = f16_to_f32(w.b[2 * b] | (w.b[2 * b + 1] << 8));
    t[0] = d * (float)(i0 + i1 - 8 * act.s[u]) * act.d[u];
  }
};

constexpr int kMvRows = 16;   // rows per block
constexpr int kMvUnits = 64;  // units per LDS chunk

// y[r] = sum of terms (or resid[r] = resid[r] + sum when resid != nullptr).
template <uint32_t TY>
__global__ void __launch_bounds__(256) k_matvec(DevMat w, Q8In act, float* y, float* resid) {
  constexpr int T = Unit<TY>::kTerms;
  __shared__ float terms[kMvRows][kMvUnits * T + 1];
  const uint32_t r0 = blockIdx.x * kMvRows;
  const uint32_t U = Unit<TY>::units(w.cols);
  float acc = 0.0f;
  for (uint32_t c0 = 0; c0 < U; c0 += kMvUnits) {
    uint32_t cn = U - c0 < (uint32_t)kMvUnits ? U - c0 : (uint32_t)kMvUnits;
    for (uint32_t idx = threadIdx.x; idx < (uint32_t)(kMvRows * kMvUnits); idx += 256) {
      uint32_t rl = idx / kMvUnits, uu = idx % kMvUnits;
      uint32_t r = r0 + rl;
      if (r < w.rows && uu < cn) Unit<TY>::run(w, act, r, c0 + uu, &terms[rl][uu * T]);
    }
    __syncthreads();
    if (threadIdx.x < (uint32_t)kMvRows) {
      const float* tr = terms[threadIdx.x];
      for (uint32_t k = 0; k < cn * T; k++) acc = acc + tr[k];
    }
    __syncthreads();
  }
  if (threadIdx.x < (uint32_t)kMvRows) {
    uint32_t r = r0 + threadIdx.x;
    if (r < w.rows) {
      if (resid)
        resid[r] = resid[r] + acc;
      else
        y[r] = acc;
    }
  }
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
      uint32_t bi = k >> 3, g = (k >> 1) & 3, hi = k & 1;
      const uint8_t* qs = w.a + (size_t)row * w.row_bytes + (size_t)bi * 144 + 16 + 32 * g;
      for (int l = 0; l < 32; l++) s += (int)((qs[l] >> (4 * hi)) & 0xF) * a[(size_t)k * 32 + l];
      break;
    }
    case RLH_TYPE_Q6_K: {  // k = 16-half index: (bi*8 + half*4 + c)*2 + sub
      uint32_t blk = k >> 1, sub = k & 1, bi = blk >> 3, half = (blk >> 2) & 1, c = blk & 3;
      size_t sbi = (size_t)row * (w.cols >> 8) + bi;
      const uint8_t* ql = w.a + sbi * 128 + half * 64 + (c & 1) * 32 + sub * 16;
      const uint8_t* qh = w.b + sbi * 64 + half * 32 + sub * 16;
      for (int l = 0; l < 16; l++) {
        uint32_t nib = c < 2 ? (ql[l] & 0xF) : (ql[l] >> 4);
        uint32_t uu = nib | (((qh[l] >> (2 * c)) & 3) << 4);
        s += (int)uu * a[(size_t)blk * 32 + sub * 16 + l];
      }
      break;
    }
    case RLH_TYPE_Q8_0: {
      const int8_t* q = (const int8_t*)(w.a + ((size_t)row * (w.cols >> 5) + k) * 32);
      for (int l = 0; l < 32; l++) s += (int)q[l] * a[(size_t)k * 32 + l];
      break;
    }
    case RLH_TYPE_Q4_0: {
      const uint8_t* q = w.a + ((size_t)row * (w.cols >> 5) + k) * 16;
      for (int l = 0; l < 16; l++) {
        s += (int)(q[l] & 0xF) * a[(size_t)k * 32 + l];
        s += (int)(q[l] >> 4) * a[(size_t)k * 32 + 16 + l];
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
// grid.x = H + KVH heads (q heads first), grid.y = tokens; block 64.
// q/k/v are token-major [n][dim]; pos of token t is pos0[0] + t.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(64) k_qk_norm_rope_kv(float* q, float* k, const float* v, const float* bq,
                                                       const float* bk, const float* bv, const float* qn,
                                                       const float* kn, const float* rope_cs, const uint32_t* pos0,
                                                       float* kcache, float* vcache, int H, int KVH, float eps) {
  constexpr int hd = 128;
  __shared__ float hbuf[hd];
  int head = blockIdx.x;
  int t = blockIdx.y;
  int lane = threadIdx.x;
  uint32_t pos = pos0[0] + (uint32_t)t;
  const int qd = H * hd, kvd = KVH * hd;
  bool is_q = head < H;
  int h = is_q ? head : head - H;
  float* src = is_q ? q + (size_t)t * qd + h * hd : k + (size_t)t * kvd + h * hd;
  const float* bias = is_q ? bq : bk;
  const float* nw = is_q ? qn : kn;
  for (int i = lane; i < hd; i += 64) {
    float x = src[i];
    if (bias) x = x + bias[h * hd + i];
    hbuf[i] = x;
  }
  __syncthreads();
  if (nw) {
    float ss = rms_sumsq_wave(hbuf, hd);
    float s = 1.0f / sqrtf(ss / (float)hd + eps);
    __syncthreads();
    for (int i = lane; i < hd; i += 64) hbuf[i] = hbuf[i] * s * nw[i];
    __syncthreads();
  }
  // RoPE pairs (i, i+64): lane i < 64 handles pair i.
  {
    int i = lane;
    float c = rope_cs[(size_t)pos * hd + 2 * i];
    float sn = rope_cs[(size_t)pos * hd + 2 * i + 1];
    float x0 = hbuf[i], x1 = hbuf[i + 64];
    float y0 = x0 * c - x1 * sn;
    float y1 = x0 * sn + x1 * c;
    if (is_q) {
      src[i] = y0;
      src[i + 64] = y1;
    } else {
      float* kd = kcache + (size_t)pos * kvd + h * hd;
      kd[i] = y0;
      kd[i + 64] = y1;
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

// ---------------------------------------------------------------------------
// Attention for one (query token, head), exact in the reference order
// (model.rs:692-711 / 525-543): s_j = dot_f32_avx2(q, K_j) * scale,
// softmax_inplace (ops.rs:398-419: sequential sum of glibc expf), then the
// saxpy chain out = (p_j * V_j) + out over j in order (simd.rs:674-691).
// Output is also quantised to Q8 (the attn_output matvec input).
// grid (H, n_tokens); block 256; dynamic LDS = t_max floats.
// Token t attends positions [0, pos0 + t].
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_attention(const float* q, const float* kcache, const float* vcache,
                                                   const uint32_t* pos0, int H, int KVH, float scale, float* out,
                                                   Q8Out out_q8) {
  constexpr int hd = 128;
  extern __shared__ float scores[];
  __shared__ float qv[hd];
  __shared__ float red[256];
  __shared__ float s_inv;
  __shared__ int s_scale_on;
  int h = blockIdx.x, tok = blockIdx.y;
  int group = H / KVH;
  if (group < 1) group = 1;
  int kvh = h / group;
  const int qd = H * hd, kvd = KVH * hd;
  uint32_t t = pos0[0] + (uint32_t)tok + 1;
  const float* qh = q + (size_t)tok * qd + h * hd;
  if (threadIdx.x < hd) qv[threadIdx.x] = qh[threadIdx.x];
  __syncthreads();
  // scores: one position per thread, the full 32-slot FMA tree in registers.
  for (uint32_t j = threadIdx.x; j < t; j += 256) {
    const float4* kr = (const float4*)(kcache + (size_t)j * kvd + kvh * hd);
    float acc[32];
#pragma unroll
    for (int s = 0; s < 32; s++) acc[s] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
      for (int s4 = 0; s4 < 8; s4++) {
        float4 kk = kr[i * 8 + s4];
        int s = s4 * 4;
        acc[s] = __builtin_fmaf(qv[i * 32 + s], kk.x, acc[s]);
        acc[s + 1] = __builtin_fmaf(qv[i * 32 + s + 1], kk.y, acc[s + 1]);
        acc[s + 2] = __builtin_fmaf(qv[i * 32 + s + 2], kk.z, acc[s + 2]);
        acc[s + 3] = __builtin_fmaf(qv[i * 32 + s + 3], kk.w, acc[s + 3]);
      }
    }
    float A[8];
#pragma unroll
    for (int l = 0; l < 8; l++) A[l] = (acc[l] + acc[8 + l]) + (acc[16 + l] + acc[24 + l]);
    float dot = ((A[0] + A[4]) + (A[2] + A[6])) + ((A[1] + A[5]) + (A[3] + A[7]));
    scores[j] = dot * scale;
  }
  __syncthreads();
  // max (order-independent)
  float mx = -__int_as_float(0x7f800000);
  for (uint32_t j = threadIdx.x; j < t; j += 256) mx = fmaxf(mx, scores[j]);
  red[threadIdx.x] = mx;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if ((int)threadIdx.x < st) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + st]);
    __syncthreads();
  }
  mx = red[0];
  for (uint32_t j = threadIdx.x; j < t; j += 256) scores[j] = expf_glibc(scores[j] - mx);
  __syncthreads();
  if (threadIdx.x == 0) {
    float sum = 0.0f;
    for (uint32_t j = 0; j < t; j++) sum = sum + scores[j];
    s_scale_on = sum > 0.0f;
    s_inv = 1.0f / sum;
  }
  __syncthreads();
  if (s_scale_on) {
    float inv = s_inv;
    for (uint32_t j = threadIdx.x; j < t; j += 256) scores[j] = scores[j] * inv;
    __syncthreads();
  }
  // saxpy chain: threads 0..127 own one output dimension each.
  float o = 0.0f;
  if (threadIdx.x < hd) {
    const float* vb = vcache + kvh * hd + threadIdx.x;
    for (uint32_t j = 0; j < t; j++) o = scores[j] * vb[(size_t)j * kvd] + o;
    out[(size_t)tok * qd + h * hd + threadIdx.x] = o;
  }
  if (threadIdx.x < hd) {
    uint32_t nbq = (uint32_t)qd / 32;
    Q8Out ot{out_q8.qs + (size_t)tok * qd, out_q8.d + (size_t)tok * nbq, out_q8.s + (size_t)tok * nbq,
             out_q8.s16 + (size_t)tok * nbq * 2};
    q8_quant_block32(o, ot, (uint32_t)(h * hd + threadIdx.x) / 32);
  }
}

// ---------------------------------------------------------------------------
// SwiGLU + Q8: h = silu(g) * u, silu(x) = x / (1 + expf(-x)) (ops.rs:393-395,
// model.rs:722-724, 565-567), then quantize_q8 of h (ffn_down input).
// grid covers n_total = n_tokens * F elements, 256 per block.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_swiglu_q8(const float* g, const float* u, uint32_t n_total, Q8Out out,
                                                   float* h_out) {
  uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (blockIdx.x * 256 + (threadIdx.x & ~31u) >= n_total) return;
  float x = g[i];
  float sl = x / (1.0f + expf_glibc(-x));
  float h = sl * u[i];
  if (h_out) h_out[i] = h;
  q8_quant_block32(h, out, i / 32);
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
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) argmax_merge(bv, bi, x[i], i);
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
// hist[++step] <- argmax.
__global__ void __launch_bounds__(256) k_argmax_final(const float* pv, const uint32_t* pi, uint32_t np,
                                                      uint32_t* tok_out, uint32_t* pos, uint32_t* step,
                                                      uint32_t* hist) {
  __shared__ float sv[256];
  __shared__ uint32_t si[256];
  float bv = -__int_as_float(0x7f800000);
  uint32_t bi = 0xffffffffu;
  for (uint32_t i = threadIdx.x; i < np; i += 256) argmax_merge(bv, bi, pv[i], pi[i]);
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if ((int)threadIdx.x < st) {
      float b = sv[threadIdx.x];
      uint32_t j = si[threadIdx.x];
      argmax_merge(b, j, sv[threadIdx.x + st], si[threadIdx.x + st]);
      sv[threadIdx.x] = b;
      si[threadIdx.x] = j;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    uint32_t best = si[0] == 0xffffffffu ? 0u : si[0];  // all NaN -> 0, as main.rs argmax
    tok_out[0] = best;
    if (step) {
      uint32_t s = step[0] + 1;
      hist[s] = best;
      step[0] = s;
      pos[0] = pos[0] + 1;
    }
  }
}

// ---------------------------------------------------------------------------
// Launch wrappers
// ---------------------------------------------------------------------------
static inline Q8In q8in(const Q8Buf& b) { return Q8In{b.qs, b.d, b.s, b.s16}; }
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
  return ty == RLH_TYPE_Q4_K || ty == RLH_TYPE_Q6_K || ty == RLH_TYPE_Q8_0 || ty == RLH_TYPE_Q4_0;
}

void launch_matvec(hipStream_t st, const DevMat& w, const Q8Buf& act, float* y, float* resid) {
  dim3 grid((w.rows + kMvRows - 1) / kMvRows);
  switch (w.ty) {
    case RLH_TYPE_Q4_K: hipLaunchKernelGGL(k_matvec<RLH_TYPE_Q4_K>, grid, dim3(256), 0, st, w, q8in(act), y, resid); break;
    case RLH_TYPE_Q6_K: hipLaunchKernelGGL(k_matvec<RLH_TYPE_Q6_K>, grid, dim3(256), 0, st, w, q8in(act), y, resid); break;
    case RLH_TYPE_Q8_0: hipLaunchKernelGGL(k_matvec<RLH_TYPE_Q8_0>, grid, dim3(256), 0, st, w, q8in(act), y, resid); break;
    case RLH_TYPE_Q4_0: hipLaunchKernelGGL(k_matvec<RLH_TYPE_Q4_0>, grid, dim3(256), 0, st, w, q8in(act), y, resid); break;
    default: break;
  }
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
  hipLaunchKernelGGL(k_qk_norm_rope_kv, dim3(H + KVH, n_tok), dim3(64), 0, st, q, k, v, bq, bk, bv, qn, kn, rope_cs,
                     pos0, kcache, vcache, H, KVH, eps);
}

void launch_attention(hipStream_t st, const float* q, const float* kcache, const float* vcache, const uint32_t* pos0,
                      int H, int KVH, uint32_t n_tok, uint32_t t_max, float scale, float* out, const Q8Buf& out_q8) {
  size_t lds = (size_t)t_max * sizeof(float);
  hipLaunchKernelGGL(k_attention, dim3(H, n_tok), dim3(256), lds, st, q, kcache, vcache, pos0, H, KVH, scale, out,
                     q8out(out_q8));
}

void launch_swiglu_q8(hipStream_t st, const float* g, const float* u, uint32_t n_total, const Q8Buf& out,
                      float* h_out) {
  hipLaunchKernelGGL(k_swiglu_q8, dim3((n_total + 255) / 256), dim3(256), 0, st, g, u, n_total, q8out(out), h_out);
}

void launch_argmax(hipStream_t st, const float* x, uint32_t n, float* pv, uint32_t* pi, uint32_t nparts,
                   uint32_t* tok_out, uint32_t* pos, uint32_t* step, uint32_t* hist) {
  hipLaunchKernelGGL(k_argmax_partial, dim3(nparts), dim3(256), 0, st, x, n, pv, pi);
  hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, st, pv, pi, nparts, tok_out, pos, step, hist);
}

}  // namespace rlh

namespace rlh {
bool attention_set_max_lds(size_t bytes) {
  return hipFuncSetAttribute((const void*)k_attention, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) ==
         hipSuccess;
}
}  // namespace rlh
