// oracle/quant_simd.cpp — restatement of src/quant.rs and src/simd.rs.
// TEST INFRASTRUCTURE ONLY (the parity oracle); never linked into librlh.so.
#include <immintrin.h>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "cpu_ref.h"
#include "internal.h"

namespace orc {

// simd.rs:17-34 — AVX2 + FMA + F16C, unless RUST_LLAMA_NO_SIMD (or ORC_NO_SIMD) is set.
bool simd_available() {
  static int state = 0;
  if (state == 0) {
    bool ok = std::getenv("RUST_LLAMA_NO_SIMD") == nullptr && std::getenv("ORC_NO_SIMD") == nullptr &&
              __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("f16c");
    state = ok ? 1 : 2;
  }
  return state == 1;
}

// quant.rs:134-157
float f16_to_f32_scalar(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t mant = h & 0x3ff;
  uint32_t bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      uint32_t e = 127 - 15 + 1;
      uint32_t m = mant;
      while ((m & 0x400) == 0) {
        m <<= 1;
        e -= 1;
      }
      bits = sign | (e << 23) | ((m & 0x3ff) << 13);
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (mant << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

__attribute__((target("f16c"))) static float f16_to_f32_f16c(uint16_t h) {
  __m128i v = _mm_cvtsi32_si128((int)h);
  __m128 f = _mm_cvtph_ps(v);
  return _mm_cvtss_f32(f);
}

// quant.rs:115-123
float f16_to_f32(uint16_t h) {
  if (simd_available()) return f16_to_f32_f16c(h);
  return f16_to_f32_scalar(h);
}

static inline float bf16_to_f32(uint16_t h) {  // quant.rs:160-162
  uint32_t b = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}
static inline float read_f16(const uint8_t* src, size_t off) {  // quant.rs:165-167
  return f16_to_f32((uint16_t)(src[off] | (src[off + 1] << 8)));
}
static inline uint32_t read_u32(const uint8_t* src, size_t off) {
  return (uint32_t)src[off] | ((uint32_t)src[off + 1] << 8) | ((uint32_t)src[off + 2] << 16) |
         ((uint32_t)src[off + 3] << 24);
}

// quant.rs:176-185
void get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
    *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

int block_size(uint32_t ty) {  // quant.rs:44-50
  switch (ty) {
    case ORC_F32: case ORC_F16: case ORC_BF16: return 1;
    case ORC_Q4_0: case ORC_Q4_1: case ORC_Q5_0: case ORC_Q5_1: case ORC_Q8_0: return 32;
    case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: return 256;
    default: return 0;
  }
}
int type_size(uint32_t ty) {  // quant.rs:53-66
  switch (ty) {
    case ORC_F32: return 4;
    case ORC_F16: case ORC_BF16: return 2;
    case ORC_Q4_0: return 18;
    case ORC_Q4_1: return 20;
    case ORC_Q5_0: return 22;
    case ORC_Q5_1: return 24;
    case ORC_Q8_0: return 34;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    default: return 0;
  }
}

// quant.rs:191-385. Rust evaluates every expression left to right with one
// rounding per operator; -ffp-contract=off keeps that here.
void dequant_row(uint32_t ty, const uint8_t* src, size_t n, float* dst) {
  switch (ty) {
    case ORC_F32:
      for (size_t i = 0; i < n; i++) std::memcpy(&dst[i], src + 4 * i, 4);
      break;
    case ORC_F16:
      for (size_t i = 0; i < n; i++) dst[i] = read_f16(src, 2 * i);
      break;
    case ORC_BF16:
      for (size_t i = 0; i < n; i++) dst[i] = bf16_to_f32((uint16_t)(src[2 * i] | (src[2 * i + 1] << 8)));
      break;
    case ORC_Q4_0:
      for (size_t bi = 0; bi < n / 32; bi++) {
        const uint8_t* block = src + bi * 18;
        float d = read_f16(block, 0);
        const uint8_t* qs = block + 2;
        size_t base = bi * 32;
        for (int j = 0; j < 16; j++) {
          float x0 = (float)((int)(qs[j] & 0x0F) - 8);
          float x1 = (float)((int)(qs[j] >> 4) - 8);
          dst[base + j] = x0 * d;
          dst[base + j + 16] = x1 * d;
        }
      }
      break;
    case ORC_Q4_1:
      for (size_t bi = 0; bi < n / 32; bi++) {
        const uint8_t* block = src + bi * 20;
        float d = read_f16(block, 0);
        float m = read_f16(block, 2);
        const uint8_t* qs = block + 4;
        size_t base = bi * 32;
        for (int j = 0; j < 16; j++) {
          float x0 = (float)(qs[j] & 0x0F);
          float x1 = (float)(qs[j] >> 4);
          dst[base + j] = x0 * d + m;
          dst[base + j + 16] = x1 * d + m;
        }
      }
      break;
    case ORC_Q5_0:
      for (size_t bi = 0; bi < n / 32; bi++) {
        const uint8_t* block = src + bi * 22;
        float d = read_f16(block, 0);
        uint32_t qh = read_u32(block, 2);
        const uint8_t* qs = block + 6;
        size_t base = bi * 32;
        for (int j = 0; j < 16; j++) {
          uint8_t xh0 = (uint8_t)(((qh >> j) << 4) & 0x10);
          uint8_t xh1 = (uint8_t)((qh >> (j + 12)) & 0x10);
          float x0 = (float)((int)((qs[j] & 0x0F) | xh0) - 16);
          float x1 = (float)((int)((qs[j] >> 4) | xh1) - 16);
          dst[base + j] = x0 * d;
          dst[base + j + 16] = x1 * d;
        }
      }
      break;
    case ORC_Q5_1:
      for (size_t bi = 0; bi < n / 32; bi++) {
        const uint8_t* block = src + bi * 24;
        float d = read_f16(block, 0);
        float m = read_f16(block, 2);
        uint32_t qh = read_u32(block, 4);
        const uint8_t* qs = block + 8;
        size_t base = bi * 32;
        for (int j = 0; j < 16; j++) {
          uint8_t xh0 = (uint8_t)(((qh >> j) << 4) & 0x10);
          uint8_t xh1 = (uint8_t)((qh >> (j + 12)) & 0x10);
          float x0 = (float)((qs[j] & 0x0F) | xh0);
          float x1 = (float)((qs[j] >> 4) | xh1);
          dst[base + j] = x0 * d + m;
          dst[base + j + 16] = x1 * d + m;
        }
      }
      break;
    case ORC_Q8_0:
      for (size_t bi = 0; bi < n / 32; bi++) {
        const uint8_t* block = src + bi * 34;
        float d = read_f16(block, 0);
        for (int j = 0; j < 32; j++) dst[bi * 32 + j] = (float)(int8_t)block[2 + j] * d;
      }
      break;
    case ORC_Q4_K:
      for (size_t bi = 0; bi < n / 256; bi++) {
        const uint8_t* block = src + bi * 144;
        float d = read_f16(block, 0);
        float dmin = read_f16(block, 2);
        const uint8_t* scales = block + 4;
        const uint8_t* qs = block + 16;
        size_t base = bi * 256;
        int is = 0;
        size_t qoff = 0;
        for (size_t yoff = base; yoff < base + 256; yoff += 64, qoff += 32, is += 2) {
          uint8_t sc1, m1, sc2, m2;
          get_scale_min_k4(is, scales, &sc1, &m1);
          get_scale_min_k4(is + 1, scales, &sc2, &m2);
          float d1 = d * (float)sc1;
          float mm1 = dmin * (float)m1;
          float d2 = d * (float)sc2;
          float mm2 = dmin * (float)m2;
          for (int l = 0; l < 32; l++) dst[yoff + l] = d1 * (float)(qs[qoff + l] & 0x0F) - mm1;
          for (int l = 0; l < 32; l++) dst[yoff + 32 + l] = d2 * (float)(qs[qoff + l] >> 4) - mm2;
        }
      }
      break;
    case ORC_Q5_K:
      for (size_t bi = 0; bi < n / 256; bi++) {
        const uint8_t* block = src + bi * 176;
        float d = read_f16(block, 0);
        float dmin = read_f16(block, 2);
        const uint8_t* scales = block + 4;
        const uint8_t* qh = block + 16;
        const uint8_t* qs = block + 48;
        size_t base = bi * 256;
        int is = 0;
        size_t qoff = 0;
        uint8_t u1 = 1, u2 = 2;
        for (size_t yoff = base; yoff < base + 256; yoff += 64, qoff += 32, is += 2) {
          uint8_t sc1, m1, sc2, m2;
          get_scale_min_k4(is, scales, &sc1, &m1);
          get_scale_min_k4(is + 1, scales, &sc2, &m2);
          float d1 = d * (float)sc1;
          float mm1 = dmin * (float)m1;
          float d2 = d * (float)sc2;
          float mm2 = dmin * (float)m2;
          for (int l = 0; l < 32; l++) {
            int hi = (qh[l] & u1) ? 16 : 0;
            dst[yoff + l] = d1 * (float)((qs[qoff + l] & 0x0F) + hi) - mm1;
          }
          for (int l = 0; l < 32; l++) {
            int hi = (qh[l] & u2) ? 16 : 0;
            dst[yoff + 32 + l] = d2 * (float)((qs[qoff + l] >> 4) + hi) - mm2;
          }
          u1 = (uint8_t)(u1 << 2);
          u2 = (uint8_t)(u2 << 2);
        }
      }
      break;
    case ORC_Q6_K:
      for (size_t bi = 0; bi < n / 256; bi++) {
        const uint8_t* block = src + bi * 210;
        float d = read_f16(block, 208);
        size_t base = bi * 256;
        size_t ql_off = 0, qh_off = 128, sc_off = 192, yoff = base;
        for (int nn = 0; nn < 256; nn += 128) {
          const uint8_t* ql = block + ql_off;
          const uint8_t* qh = block + qh_off;
          const int8_t* sc = (const int8_t*)(block + sc_off);
          for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            dst[yoff + l] = d * (float)sc[is] * (float)q1;
            dst[yoff + l + 32] = d * (float)sc[is + 2] * (float)q2;
            dst[yoff + l + 64] = d * (float)sc[is + 4] * (float)q3;
            dst[yoff + l + 96] = d * (float)sc[is + 6] * (float)q4;
          }
          yoff += 128;
          ql_off += 64;
          qh_off += 32;
          sc_off += 8;
        }
      }
      break;
    default:
      break;
  }
}

float dot_scalar(const float* a, const float* b, size_t n);  // ops.cpp

// quant.rs:409-541
float dequant_dot_scalar(uint32_t ty, const uint8_t* src, const float* x, size_t n) {
  switch (ty) {
    case ORC_F32: {
      float acc = 0.f;
      for (size_t i = 0; i < n; i++) {
        float w;
        std::memcpy(&w, src + 4 * i, 4);
        acc += w * x[i];
      }
      return acc;
    }
    case ORC_F16: {
      float acc = 0.f;
      for (size_t i = 0; i < n; i++) acc += read_f16(src, 2 * i) * x[i];
      return acc;
    }
    case ORC_BF16: {
      float acc = 0.f;
      for (size_t i = 0; i < n; i++) acc += bf16_to_f32((uint16_t)(src[2 * i] | (src[2 * i + 1] << 8))) * x[i];
      return acc;
    }
    case ORC_Q4_0: {
      float acc = 0.f;
      for (size_t bi = 0; bi < n / 32; bi++) {
        const uint8_t* block = src + bi * 18;
        float d = read_f16(block, 0);
        const uint8_t* qs = block + 2;
        const float* xb = x + bi * 32;
        float s = 0.f;
        for (int j = 0; j < 16; j++) {
          float x0 = (float)((int)(qs[j] & 0x0F) - 8);
          float x1 = (float)((int)(qs[j] >> 4) - 8);
          s += x0 * xb[j] + x1 * xb[j + 16];
        }
        acc += d * s;
      }
      return acc;
    }
    case ORC_Q8_0: {
      float acc = 0.f;
      for (size_t bi = 0; bi < n / 32; bi++) {
        const uint8_t* block = src + bi * 34;
        float d = read_f16(block, 0);
        const float* xb = x + bi * 32;
        float s = 0.f;
        for (int j = 0; j < 32; j++) s += (float)(int8_t)block[2 + j] * xb[j];
        acc += d * s;
      }
      return acc;
    }
    case ORC_Q4_K: {
      float acc = 0.f;
      for (size_t bi = 0; bi < n / 256; bi++) {
        const uint8_t* block = src + bi * 144;
        float d = read_f16(block, 0);
        float dmin = read_f16(block, 2);
        const uint8_t* scales = block + 4;
        const uint8_t* qs = block + 16;
        const float* xb = x + bi * 256;
        int is = 0;
        size_t qoff = 0;
        float s = 0.f;
        for (size_t yoff = 0; yoff < 256; yoff += 64, qoff += 32, is += 2) {
          uint8_t sc1, m1, sc2, m2;
          get_scale_min_k4(is, scales, &sc1, &m1);
          get_scale_min_k4(is + 1, scales, &sc2, &m2);
          float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
          float d2 = d * (float)sc2, mm2 = dmin * (float)m2;
          for (int l = 0; l < 32; l++) {
            s += (d1 * (float)(qs[qoff + l] & 0x0F) - mm1) * xb[yoff + l];
            s += (d2 * (float)(qs[qoff + l] >> 4) - mm2) * xb[yoff + 32 + l];
          }
        }
        acc += s;
      }
      return acc;
    }
    case ORC_Q6_K: {
      float acc = 0.f;
      for (size_t bi = 0; bi < n / 256; bi++) {
        const uint8_t* block = src + bi * 210;
        float d = read_f16(block, 208);
        const float* xb = x + bi * 256;
        size_t ql_off = 0, qh_off = 128, sc_off = 192, yoff = 0;
        for (int nn = 0; nn < 256; nn += 128) {
          const uint8_t* ql = block + ql_off;
          const uint8_t* qh = block + qh_off;
          const int8_t* sc = (const int8_t*)(block + sc_off);
          for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)((ql[l] & 0x0F) | ((qh[l] & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            acc += d * (float)sc[is] * (float)q1 * xb[yoff + l];
            acc += d * (float)sc[is + 2] * (float)q2 * xb[yoff + l + 32];
            acc += d * (float)sc[is + 4] * (float)q3 * xb[yoff + l + 64];
            acc += d * (float)sc[is + 6] * (float)q4 * xb[yoff + l + 96];
          }
          yoff += 128;
          ql_off += 64;
          qh_off += 32;
          sc_off += 8;
        }
      }
      return acc;
    }
    default: {  // quant.rs:528-539 generic fallback, one block at a time
      int bs = block_size(ty), ts = type_size(ty);
      if (bs == 0) return 0.f;
      float tmp[256];
      float acc = 0.f;
      for (size_t bi = 0; bi < n / bs; bi++) {
        dequant_row(ty, src + bi * ts, (size_t)bs, tmp);
        acc += dot(tmp, x + bi * bs, (size_t)bs);
      }
      return acc;
    }
  }
}

// ---------------------------------------------------------------------------
// AVX2 kernels (simd.rs). Same intrinsics, same order.
// ---------------------------------------------------------------------------
#define AVX2_FN __attribute__((target("avx2,fma,f16c")))

// simd.rs:261-270
AVX2_FN static inline float hsum(__m256 v) {
  __m128 lo = _mm256_castps256_ps128(v);
  __m128 hi = _mm256_extractf128_ps(v, 1);
  __m128 s = _mm_add_ps(lo, hi);
  __m128 hi64 = _mm_movehl_ps(s, s);
  __m128 s2 = _mm_add_ps(s, hi64);
  __m128 hi32 = _mm_shuffle_ps(s2, s2, 0x55);
  __m128 s3 = _mm_add_ss(s2, hi32);
  return _mm_cvtss_f32(s3);
}
// simd.rs:525-534
AVX2_FN static inline int32_t hsum_i32(__m256i v) {
  __m128i lo = _mm256_castsi256_si128(v);
  __m128i hi = _mm256_extracti128_si256(v, 1);
  __m128i s = _mm_add_epi32(lo, hi);
  __m128i hi64 = _mm_shuffle_epi32(s, 0xee);
  __m128i s2 = _mm_add_epi32(s, hi64);
  __m128i hi32 = _mm_shuffle_epi32(s2, 0x55);
  __m128i s3 = _mm_add_epi32(s2, hi32);
  return _mm_cvtsi128_si32(s3);
}
// simd.rs:590-596
AVX2_FN static inline int32_t hsum_i32_128(__m128i v) {
  __m128i hi64 = _mm_shuffle_epi32(v, 0xee);
  __m128i s = _mm_add_epi32(v, hi64);
  __m128i hi32 = _mm_shuffle_epi32(s, 0x55);
  __m128i s2 = _mm_add_epi32(s, hi32);
  return _mm_cvtsi128_si32(s2);
}
static inline float f16_at(const uint8_t* p) { return f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

// simd.rs:116-203
AVX2_FN void quantize_q8_avx2(const float* x, size_t n, int8_t* qs, float* scales, int32_t* sums,
                              int32_t* sums16) {
  size_t nb = n / 32;
  const __m256 sign_mask = _mm256_set1_ps(-0.0f);
  const __m128i ones = _mm_set1_epi16(1);
  for (size_t b = 0; b < nb; b++) {
    const float* blk = x + b * 32;
    __m256 v0 = _mm256_loadu_ps(blk), v1 = _mm256_loadu_ps(blk + 8);
    __m256 v2 = _mm256_loadu_ps(blk + 16), v3 = _mm256_loadu_ps(blk + 24);
    __m256 abs0 = _mm256_andnot_ps(sign_mask, v0), abs1 = _mm256_andnot_ps(sign_mask, v1);
    __m256 abs2 = _mm256_andnot_ps(sign_mask, v2), abs3 = _mm256_andnot_ps(sign_mask, v3);
    __m256 max01 = _mm256_max_ps(abs0, abs1);
    __m256 max23 = _mm256_max_ps(abs2, abs3);
    __m256 max_all = _mm256_max_ps(max01, max23);
    __m128 max_lo = _mm256_castps256_ps128(max_all);
    __m128 max_hi = _mm256_extractf128_ps(max_all, 1);
    __m128 max_128 = _mm_max_ps(max_lo, max_hi);
    __m128 max_64 = _mm_max_ps(max_128, _mm_movehl_ps(max_128, max_128));
    __m128 max_32 = _mm_max_ss(max_64, _mm_shuffle_ps(max_64, max_64, 0x55));
    float amax = _mm_cvtss_f32(max_32);
    float d = amax / 127.0f;
    float inv = d > 0.0f ? 1.0f / d : 0.0f;
    scales[b] = d;
    __m256 inv_v = _mm256_set1_ps(inv);
    __m256i q0 = _mm256_cvtps_epi32(_mm256_mul_ps(v0, inv_v));
    __m256i q1 = _mm256_cvtps_epi32(_mm256_mul_ps(v1, inv_v));
    __m256i q2 = _mm256_cvtps_epi32(_mm256_mul_ps(v2, inv_v));
    __m256i q3 = _mm256_cvtps_epi32(_mm256_mul_ps(v3, inv_v));
    __m256i pack01 = _mm256_packs_epi32(q0, q1);
    __m256i pack23 = _mm256_packs_epi32(q2, q3);
    __m256i pack01_perm = _mm256_permute4x64_epi64(pack01, 0xd8);
    __m256i pack23_perm = _mm256_permute4x64_epi64(pack23, 0xd8);
    __m256i pack_all = _mm256_packs_epi16(pack01_perm, pack23_perm);
    __m256i pack_all_perm = _mm256_permute4x64_epi64(pack_all, 0xd8);
    _mm256_storeu_si256((__m256i*)(qs + b * 32), pack_all_perm);
    __m128i lo128 = _mm256_castsi256_si128(pack_all_perm);
    __m128i hi128 = _mm256_extracti128_si256(pack_all_perm, 1);
    __m128i s_lo_16 = _mm_maddubs_epi16(_mm_set1_epi8(1), lo128);
    __m128i s_lo_32 = _mm_madd_epi16(s_lo_16, ones);
    __m128i hi64 = _mm_shuffle_epi32(s_lo_32, 0xee);
    __m128i s_32 = _mm_add_epi32(s_lo_32, hi64);
    int32_t s_lo = _mm_cvtsi128_si32(_mm_add_epi32(s_32, _mm_shuffle_epi32(s_32, 0x55)));
    __m128i s_hi_16 = _mm_maddubs_epi16(_mm_set1_epi8(1), hi128);
    __m128i s_hi_32 = _mm_madd_epi16(s_hi_16, ones);
    __m128i hi64_h = _mm_shuffle_epi32(s_hi_32, 0xee);
    __m128i s_32_h = _mm_add_epi32(s_hi_32, hi64_h);
    int32_t s_hi = _mm_cvtsi128_si32(_mm_add_epi32(s_32_h, _mm_shuffle_epi32(s_32_h, 0x55)));
    sums[b] = s_lo + s_hi;
    sums16[2 * b] = s_lo;
    sums16[2 * b + 1] = s_hi;
  }
}

// Rust `f32 as i8`: saturating, NaN -> 0.
static inline int8_t f32_as_i8(float v) {
  if (std::isnan(v)) return 0;
  if (v >= 127.f) return 127;
  if (v <= -128.f) return -128;
  return (int8_t)v;
}

// simd.rs:206-244 (f32::round = round half away from zero)
void quantize_q8_scalar(const float* x, size_t n, int8_t* qs, float* scales, int32_t* sums,
                        int32_t* sums16) {
  size_t nb = n / 32;
  for (size_t b = 0; b < nb; b++) {
    const float* blk = x + b * 32;
    float amax = 0.f;
    for (int i = 0; i < 32; i++) {
      float a = std::fabs(blk[i]);
      if (a > amax) amax = a;
    }
    float d = amax / 127.0f;
    float inv = d > 0.0f ? 1.0f / d : 0.0f;
    scales[b] = d;
    int32_t s = 0, s_lo = 0;
    for (int i = 0; i < 32; i++) {
      float r = std::round(blk[i] * inv);
      float c = std::isnan(r) ? r : std::fmin(std::fmax(r, -128.0f), 127.0f);
      int8_t q = f32_as_i8(c);
      s += q;
      if (i < 16) s_lo += q;
      qs[b * 32 + i] = q;
    }
    sums[b] = s;
    sums16[2 * b] = s_lo;
    sums16[2 * b + 1] = s - s_lo;
  }
}

// simd.rs:282-326
AVX2_FN void rmsnorm_core(float* out, const float* x, const float* w, size_t n, float eps) {
  __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps(), a2 = _mm256_setzero_ps(), a3 = _mm256_setzero_ps();
  size_t i = 0;
  while (i + 32 <= n) {
    __m256 v0 = _mm256_loadu_ps(x + i), v1 = _mm256_loadu_ps(x + i + 8);
    __m256 v2 = _mm256_loadu_ps(x + i + 16), v3 = _mm256_loadu_ps(x + i + 24);
    a0 = _mm256_fmadd_ps(v0, v0, a0);
    a1 = _mm256_fmadd_ps(v1, v1, a1);
    a2 = _mm256_fmadd_ps(v2, v2, a2);
    a3 = _mm256_fmadd_ps(v3, v3, a3);
    i += 32;
  }
  while (i + 8 <= n) {
    __m256 v = _mm256_loadu_ps(x + i);
    a0 = _mm256_fmadd_ps(v, v, a0);
    i += 8;
  }
  float ss = hsum(_mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3)));
  while (i < n) {
    float v = x[i];
    ss += v * v;
    i++;
  }
  float s = 1.0f / std::sqrt(ss / (float)n + eps);
  __m256 sv = _mm256_set1_ps(s);
  size_t j = 0;
  while (j + 8 <= n) {
    __m256 v = _mm256_mul_ps(_mm256_loadu_ps(x + j), sv);
    _mm256_storeu_ps(out + j, _mm256_mul_ps(v, _mm256_loadu_ps(w + j)));
    j += 8;
  }
  while (j < n) {
    out[j] = x[j] * s * w[j];
    j++;
  }
}

// simd.rs:328-377
AVX2_FN float dot_f32_avx2(const float* a, const float* b, size_t n) {
  __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps(), a2 = _mm256_setzero_ps(), a3 = _mm256_setzero_ps();
  size_t i = 0;
  while (i + 32 <= n) {
    a0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), a0);
    a1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), a1);
    a2 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 16), _mm256_loadu_ps(b + i + 16), a2);
    a3 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 24), _mm256_loadu_ps(b + i + 24), a3);
    i += 32;
  }
  while (i + 8 <= n) {
    a0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), a0);
    i += 8;
  }
  __m256 acc = _mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3));
  float s = hsum(acc);
  while (i < n) {
    s += a[i] * b[i];
    i++;
  }
  return s;
}

// simd.rs:380-399
AVX2_FN static float f32_bytes_avx2(const uint8_t* src, const float* x, size_t n) {
  __m256 acc = _mm256_setzero_ps();
  size_t i = 0;
  while (i + 8 <= n) {
    __m256 v = _mm256_castsi256_ps(_mm256_loadu_si256((const __m256i*)(src + i * 4)));
    acc = _mm256_fmadd_ps(v, _mm256_loadu_ps(x + i), acc);
    i += 8;
  }
  float s = hsum(acc);
  while (i < n) {
    float v;
    std::memcpy(&v, src + 4 * i, 4);
    s += v * x[i];
    i++;
  }
  return s;
}

// simd.rs:401-419
AVX2_FN static float f16_avx2(const uint8_t* src, const float* x, size_t n) {
  __m256 acc = _mm256_setzero_ps();
  size_t i = 0;
  while (i + 8 <= n) {
    __m128i h = _mm_loadu_si128((const __m128i*)(src + i * 2));
    __m256 v = _mm256_cvtph_ps(h);
    acc = _mm256_fmadd_ps(v, _mm256_loadu_ps(x + i), acc);
    i += 8;
  }
  float s = hsum(acc);
  while (i < n) {
    s += f16_to_f32((uint16_t)(src[2 * i] | (src[2 * i + 1] << 8))) * x[i];
    i++;
  }
  return s;
}

// simd.rs:421-448
AVX2_FN static float q4_0_avx2(const uint8_t* src, const float* x, size_t n) {
  const __m128i m0f = _mm_set1_epi8(0x0F);
  const __m256 c8 = _mm256_set1_ps(8.0f);
  float total = 0.f;
  for (size_t bi = 0; bi < n / 32; bi++) {
    size_t base = bi * 18;
    float d = f16_at(src + base);
    const uint8_t* qs = src + base + 2;
    const float* xp = x + bi * 32;
    __m256 a_lo = _mm256_setzero_ps(), a_hi = _mm256_setzero_ps();
    for (int k = 0; k < 2; k++) {
      __m128i b = _mm_loadl_epi64((const __m128i*)(qs + k * 8));
      __m128i lo = _mm_and_si128(b, m0f);
      __m128i hi = _mm_and_si128(_mm_srli_epi16(b, 4), m0f);
      __m256 lof = _mm256_sub_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(lo)), c8);
      __m256 hif = _mm256_sub_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(hi)), c8);
      a_lo = _mm256_fmadd_ps(lof, _mm256_loadu_ps(xp + k * 8), a_lo);
      a_hi = _mm256_fmadd_ps(hif, _mm256_loadu_ps(xp + 16 + k * 8), a_hi);
    }
    total += d * hsum(_mm256_add_ps(a_lo, a_hi));
  }
  return total;
}

// simd.rs:450-470
AVX2_FN static float q8_0_avx2(const uint8_t* src, const float* x, size_t n) {
  float total = 0.f;
  for (size_t bi = 0; bi < n / 32; bi++) {
    size_t base = bi * 34;
    float d = f16_at(src + base);
    const int8_t* qs = (const int8_t*)(src + base + 2);
    const float* xp = x + bi * 32;
    __m256 acc = _mm256_setzero_ps();
    for (int k = 0; k < 4; k++) {
      __m128i b = _mm_loadl_epi64((const __m128i*)(qs + k * 8));
      __m256 v = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(b));
      acc = _mm256_fmadd_ps(v, _mm256_loadu_ps(xp + k * 8), acc);
    }
    total += d * hsum(acc);
  }
  return total;
}

// simd.rs:472-520
AVX2_FN static float q4k_avx2(const uint8_t* src, const float* x, size_t n) {
  const __m128i m0f = _mm_set1_epi8(0x0F);
  float total = 0.f;
  for (size_t bi = 0; bi < n / 256; bi++) {
    size_t base = bi * 144;
    float d = f16_at(src + base);
    float dmin = f16_at(src + base + 2);
    const uint8_t* scales = src + base + 4;
    const uint8_t* qs = src + base + 16;
    const float* xp = x + bi * 256;
    float block_dot = 0.f;
    for (int g = 0; g < 4; g++) {
      uint8_t sc1, m1, sc2, m2;
      get_scale_min_k4(2 * g, scales, &sc1, &m1);
      get_scale_min_k4(2 * g + 1, scales, &sc2, &m2);
      float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
      float d2 = d * (float)sc2, mm2 = dmin * (float)m2;
      const uint8_t* qsg = qs + g * 32;
      const float* xlo = xp + g * 64;
      const float* xhi = xp + g * 64 + 32;
      __m256 sq_lo = _mm256_setzero_ps(), sq_hi = _mm256_setzero_ps();
      __m256 sx_lo = _mm256_setzero_ps(), sx_hi = _mm256_setzero_ps();
      for (int k = 0; k < 4; k++) {
        __m128i b = _mm_loadl_epi64((const __m128i*)(qsg + k * 8));
        __m128i lo = _mm_and_si128(b, m0f);
        __m128i hi = _mm_and_si128(_mm_srli_epi16(b, 4), m0f);
        __m256 lof = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(lo));
        __m256 hif = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(hi));
        __m256 vlo = _mm256_loadu_ps(xlo + k * 8);
        __m256 vhi = _mm256_loadu_ps(xhi + k * 8);
        sq_lo = _mm256_fmadd_ps(lof, vlo, sq_lo);
        sq_hi = _mm256_fmadd_ps(hif, vhi, sq_hi);
        sx_lo = _mm256_add_ps(sx_lo, vlo);
        sx_hi = _mm256_add_ps(sx_hi, vhi);
      }
      block_dot += d1 * hsum(sq_lo) - mm1 * hsum(sx_lo) + d2 * hsum(sq_hi) - mm2 * hsum(sx_hi);
    }
    total += block_dot;
  }
  return total;
}

// simd.rs:971-1048
AVX2_FN static float q6k_avx2(const uint8_t* src, const float* x, size_t n) {
  const __m128i m0f = _mm_set1_epi8(0x0F);
  const __m128i m03 = _mm_set1_epi8(0x03);
  const __m256 c32 = _mm256_set1_ps(32.0f);
  float total = 0.f;
  for (size_t bi = 0; bi < n / 256; bi++) {
    size_t base = bi * 210;
    float d = f16_at(src + base + 208);
    const float* xp = x + bi * 256;
    float block_dot = 0.f;
    size_t yoff = 0, ql_off = 0, qh_off = 128, sc_off = 192;
    for (int nn = 0; nn < 256; nn += 128) {
      for (int half = 0; half < 2; half++) {
        int is = half;
        float s1 = (float)(int8_t)src[base + sc_off + is];
        float s2 = (float)(int8_t)src[base + sc_off + is + 2];
        float s3 = (float)(int8_t)src[base + sc_off + is + 4];
        float s4 = (float)(int8_t)src[base + sc_off + is + 6];
        __m256 a1 = _mm256_setzero_ps(), a2 = _mm256_setzero_ps(), a3 = _mm256_setzero_ps(), a4 = _mm256_setzero_ps();
        for (int k = 0; k < 2; k++) {
          size_t l = (size_t)half * 16 + (size_t)k * 8;
          const uint8_t* ql = src + base + ql_off + l;
          const uint8_t* qh = src + base + qh_off + l;
          __m128i b0 = _mm_loadl_epi64((const __m128i*)ql);
          __m128i b1 = _mm_loadl_epi64((const __m128i*)(ql + 32));
          __m128i h = _mm_loadl_epi64((const __m128i*)qh);
          __m128i n0 = _mm_and_si128(b0, m0f);
          __m128i n1 = _mm_and_si128(b1, m0f);
          __m128i n2 = _mm_and_si128(_mm_srli_epi16(b0, 4), m0f);
          __m128i n3 = _mm_and_si128(_mm_srli_epi16(b1, 4), m0f);
          __m128i h0 = _mm_slli_epi16(_mm_and_si128(h, m03), 4);
          __m128i h1 = _mm_slli_epi16(_mm_and_si128(_mm_srli_epi16(h, 2), m03), 4);
          __m128i h2 = _mm_slli_epi16(_mm_and_si128(_mm_srli_epi16(h, 4), m03), 4);
          __m128i h3 = _mm_slli_epi16(_mm_and_si128(_mm_srli_epi16(h, 6), m03), 4);
          __m256 f1 = _mm256_sub_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_or_si128(n0, h0))), c32);
          __m256 f2 = _mm256_sub_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_or_si128(n1, h1))), c32);
          __m256 f3 = _mm256_sub_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_or_si128(n2, h2))), c32);
          __m256 f4 = _mm256_sub_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_or_si128(n3, h3))), c32);
          a1 = _mm256_fmadd_ps(f1, _mm256_loadu_ps(xp + yoff + l), a1);
          a2 = _mm256_fmadd_ps(f2, _mm256_loadu_ps(xp + yoff + l + 32), a2);
          a3 = _mm256_fmadd_ps(f3, _mm256_loadu_ps(xp + yoff + l + 64), a3);
          a4 = _mm256_fmadd_ps(f4, _mm256_loadu_ps(xp + yoff + l + 96), a4);
        }
        block_dot += d * (s1 * hsum(a1) + s2 * hsum(a2) + s3 * hsum(a3) + s4 * hsum(a4));
      }
      yoff += 128;
      ql_off += 64;
      qh_off += 32;
      sc_off += 8;
    }
    total += block_dot;
  }
  return total;
}

// simd.rs:38-51 + 248-257: AVX2 fused dequant-dot for the types that have one.
bool dequant_dot_avx2(uint32_t ty, const uint8_t* src, const float* x, size_t n, float* out) {
  if (!simd_available()) return false;
  switch (ty) {
    case ORC_Q4_K: *out = q4k_avx2(src, x, n); return true;
    case ORC_Q6_K: *out = q6k_avx2(src, x, n); return true;
    case ORC_Q8_0: *out = q8_0_avx2(src, x, n); return true;
    case ORC_Q4_0: *out = q4_0_avx2(src, x, n); return true;
    case ORC_F16: *out = f16_avx2(src, x, n); return true;
    case ORC_F32: *out = f32_bytes_avx2(src, x, n); return true;
    default: return false;
  }
}

// simd.rs:544-585
AVX2_FN static float dot_q4k_q8_avx2(const uint8_t* src, size_t n, const Q8View& act) {
  size_t n256 = n / 256;
  const __m256i m0f = _mm256_set1_epi8(0x0F);
  const __m256i ones = _mm256_set1_epi16(1);
  float total = 0.f;
  for (size_t bi = 0; bi < n256; bi++) {
    size_t base = bi * 144;
    float d = f16_at(src + base);
    float dmin = f16_at(src + base + 2);
    const uint8_t* scales = src + base + 4;
    const uint8_t* qs = src + base + 16;
    for (int g = 0; g < 4; g++) {
      uint8_t sc1, m1, sc2, m2;
      get_scale_min_k4(2 * g, scales, &sc1, &m1);
      get_scale_min_k4(2 * g + 1, scales, &sc2, &m2);
      float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
      float d2 = d * (float)sc2, mm2 = dmin * (float)m2;
      size_t ab = bi * 8 + 2 * g;
      float sa = (float)act.sums[ab];
      float sb = (float)act.sums[ab + 1];
      float da = act.scales[ab];
      float db = act.scales[ab + 1];
      __m256i p = _mm256_loadu_si256((const __m256i*)(qs + g * 32));
      __m256i lo = _mm256_and_si256(p, m0f);
      __m256i hi = _mm256_and_si256(_mm256_srli_epi16(p, 4), m0f);
      __m256i a = _mm256_loadu_si256((const __m256i*)(act.qs + ab * 32));
      __m256i b = _mm256_loadu_si256((const __m256i*)(act.qs + (ab + 1) * 32));
      __m256i s1 = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, a), ones);
      __m256i s2 = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, b), ones);
      float i1 = (float)hsum_i32(s1);
      float i2 = (float)hsum_i32(s2);
      total += da * (d1 * i1 - mm1 * sa) + db * (d2 * i2 - mm2 * sb);
    }
  }
  return total;
}

// simd.rs:605-669
AVX2_FN static float dot_q6k_q8_avx2(const uint8_t* src, size_t n, const Q8View& act) {
  size_t n256 = n / 256;
  const __m128i m0f = _mm_set1_epi8(0x0F);
  const __m128i m03 = _mm_set1_epi8(0x03);
  const __m128i ones = _mm_set1_epi16(1);
  float total = 0.f;
  for (size_t bi = 0; bi < n256; bi++) {
    size_t base = bi * 210;
    float d = f16_at(src + base + 208);
    for (int half = 0; half < 2; half++) {
      const uint8_t* ql = src + base + half * 64;
      const uint8_t* qh = src + base + 128 + half * 32;
      const uint8_t* sc = src + base + 192 + half * 8;
      size_t ab = bi * 8 + half * 4;
      for (int sub = 0; sub < 2; sub++) {
        int o = sub * 16;
        float scs[4] = {(float)(int8_t)sc[sub], (float)(int8_t)sc[sub + 2], (float)(int8_t)sc[sub + 4],
                        (float)(int8_t)sc[sub + 6]};
        __m128i ql0 = _mm_loadu_si128((const __m128i*)(ql + o));
        __m128i ql1 = _mm_loadu_si128((const __m128i*)(ql + 32 + o));
        __m128i qh16 = _mm_loadu_si128((const __m128i*)(qh + o));
        __m128i us[4];
        us[0] = _mm_or_si128(_mm_and_si128(ql0, m0f), _mm_slli_epi16(_mm_and_si128(qh16, m03), 4));
        us[1] = _mm_or_si128(_mm_and_si128(ql1, m0f),
                             _mm_slli_epi16(_mm_and_si128(_mm_srli_epi16(qh16, 2), m03), 4));
        us[2] = _mm_or_si128(_mm_and_si128(_mm_srli_epi16(ql0, 4), m0f),
                             _mm_slli_epi16(_mm_and_si128(_mm_srli_epi16(qh16, 4), m03), 4));
        us[3] = _mm_or_si128(_mm_and_si128(_mm_srli_epi16(ql1, 4), m0f),
                             _mm_slli_epi16(_mm_and_si128(_mm_srli_epi16(qh16, 6), m03), 4));
        const int8_t* aq = act.qs;
        __m128i aa[4];
        for (int c = 0; c < 4; c++) aa[c] = _mm_loadu_si128((const __m128i*)(aq + (ab + c) * 32 + o));
        for (int c = 0; c < 4; c++) {
          int32_t ss = hsum_i32_128(_mm_madd_epi16(_mm_maddubs_epi16(us[c], aa[c]), ones));
          int32_t sa = act.sums16[(ab + c) * 2 + sub];
          float da = act.scales[ab + c];
          total += d * scs[c] * ((float)ss - 32.0f * (float)sa) * da;
        }
      }
    }
  }
  return total;
}

// simd.rs:844-866
AVX2_FN static float dot_q40_q8_avx2(const uint8_t* src, size_t n, const Q8View& act) {
  const __m128i m0f = _mm_set1_epi8(0x0F);
  const __m128i ones = _mm_set1_epi16(1);
  float total = 0.f;
  for (size_t bi = 0; bi < n / 32; bi++) {
    size_t base = bi * 18;
    float d = f16_at(src + base);
    __m128i b = _mm_loadu_si128((const __m128i*)(src + base + 2));
    __m128i lo = _mm_and_si128(b, m0f);
    __m128i hi = _mm_and_si128(_mm_srli_epi16(b, 4), m0f);
    __m128i a0 = _mm_loadu_si128((const __m128i*)(act.qs + bi * 32));
    __m128i a1 = _mm_loadu_si128((const __m128i*)(act.qs + bi * 32 + 16));
    __m128i s0 = _mm_madd_epi16(_mm_maddubs_epi16(lo, a0), ones);
    __m128i s1 = _mm_madd_epi16(_mm_maddubs_epi16(hi, a1), ones);
    int32_t i0 = hsum_i32_128(s0);
    int32_t i1 = hsum_i32_128(s1);
    total += d * (float)(i0 + i1 - 8 * act.sums[bi]) * act.scales[bi];
  }
  return total;
}

// simd.rs:874-894
AVX2_FN static float dot_q80_q8_avx2(const uint8_t* src, size_t n, const Q8View& act) {
  float total = 0.f;
  for (size_t bi = 0; bi < n / 32; bi++) {
    size_t base = bi * 34;
    float d = f16_at(src + base);
    const uint8_t* w = src + base + 2;
    const int8_t* a = act.qs + bi * 32;
    __m256i acc = _mm256_setzero_si256();
    for (int k = 0; k < 2; k++) {
      __m128i w16 = _mm_loadu_si128((const __m128i*)(w + k * 16));
      __m128i a16 = _mm_loadu_si128((const __m128i*)(a + k * 16));
      __m256i w32 = _mm256_cvtepi8_epi16(w16);
      __m256i a32 = _mm256_cvtepi8_epi16(a16);
      acc = _mm256_add_epi32(acc, _mm256_madd_epi16(w32, a32));
    }
    total += d * (float)hsum_i32(acc) * act.scales[bi];
  }
  return total;
}

// simd.rs:898-910
bool dot_qk_q8_row(uint32_t ty, const uint8_t* src, size_t n, const Q8View& act, float* out) {
  if (!simd_available()) return false;
  switch (ty) {
    case ORC_Q4_K: *out = dot_q4k_q8_avx2(src, n, act); return true;
    case ORC_Q6_K: *out = dot_q6k_q8_avx2(src, n, act); return true;
    case ORC_Q4_0: *out = dot_q40_q8_avx2(src, n, act); return true;
    case ORC_Q8_0: *out = dot_q80_q8_avx2(src, n, act); return true;
    default: return false;
  }
}

// simd.rs:674-691 (mul then add, never FMA)
AVX2_FN void saxpy_avx2(float* dst, float alpha, const float* x, size_t n) {
  __m256 a = _mm256_set1_ps(alpha);
  size_t i = 0;
  while (i + 8 <= n) {
    __m256 d = _mm256_loadu_ps(dst + i);
    __m256 v = _mm256_loadu_ps(x + i);
    _mm256_storeu_ps(dst + i, _mm256_add_ps(_mm256_mul_ps(a, v), d));
    i += 8;
  }
  while (i < n) {
    dst[i] += alpha * x[i];
    i++;
  }
}

// simd.rs:702-754
AVX2_FN void dot_multi(const float* buf, size_t cols, const float* xs, size_t xs_off, size_t xs_stride,
                       size_t n, float* out, size_t out_stride) {
  size_t k = 0;
  while (k + 4 <= n) {
    const float* x0 = xs + k * xs_stride + xs_off;
    const float* x1 = xs + (k + 1) * xs_stride + xs_off;
    const float* x2 = xs + (k + 2) * xs_stride + xs_off;
    const float* x3 = xs + (k + 3) * xs_stride + xs_off;
    __m256 v0 = _mm256_setzero_ps(), v1 = _mm256_setzero_ps(), v2 = _mm256_setzero_ps(), v3 = _mm256_setzero_ps();
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    size_t i = 0;
    while (i + 8 <= cols) {
      __m256 w = _mm256_loadu_ps(buf + i);
      v0 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x0 + i), v0);
      v1 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x1 + i), v1);
      v2 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x2 + i), v2);
      v3 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x3 + i), v3);
      i += 8;
    }
    while (i < cols) {
      float w = buf[i];
      a0 += w * x0[i];
      a1 += w * x1[i];
      a2 += w * x2[i];
      a3 += w * x3[i];
      i++;
    }
    out[k * out_stride] += hsum(v0) + a0;
    out[(k + 1) * out_stride] += hsum(v1) + a1;
    out[(k + 2) * out_stride] += hsum(v2) + a2;
    out[(k + 3) * out_stride] += hsum(v3) + a3;
    k += 4;
  }
  while (k < n) {
    const float* xk = xs + k * xs_stride + xs_off;
    out[k * out_stride] += dot_f32_avx2(buf, xk, cols);
    k++;
  }
}

// simd.rs:782-836 with RB = 3, TB = 4 (the split matmul_batch ships, ops.rs:252-253)
AVX2_FN void dot_multi_rows_3_4(const float* bufs, size_t cols, const float* xs, size_t n, size_t cnt,
                                float* out, size_t out_stride) {
  constexpr size_t RB = 3, TB = 4;
  size_t k = 0;
  while (k + TB <= n) {
    __m256 acc[RB][TB];
    for (size_t r = 0; r < RB; r++)
      for (size_t t = 0; t < TB; t++) acc[r][t] = _mm256_setzero_ps();
    size_t i = 0;
    while (i + 8 <= cols) {
      __m256 xv[TB];
      for (size_t t = 0; t < TB; t++) xv[t] = _mm256_loadu_ps(xs + (k + t) * cols + i);
      for (size_t r = 0; r < RB; r++) {
        __m256 w = _mm256_loadu_ps(bufs + r * cols + i);
        for (size_t t = 0; t < TB; t++) acc[r][t] = _mm256_fmadd_ps(w, xv[t], acc[r][t]);
      }
      i += 8;
    }
    for (size_t r = 0; r < cnt; r++) {
      for (size_t t = 0; t < TB; t++) {
        float a = 0.f;
        for (size_t j = i; j < cols; j++) a += bufs[r * cols + j] * xs[(k + t) * cols + j];
        out[(k + t) * out_stride + r] += hsum(acc[r][t]) + a;
      }
    }
    k += TB;
  }
  while (k < n) {
    for (size_t r = 0; r < cnt; r++) out[k * out_stride + r] += dot_f32_avx2(bufs + r * cols, xs + k * cols, cols);
    k++;
  }
}

// simd.rs:918-958 (split Q4_K dequant: sub_mul = a*b - c, lane-wise, no FMA)
AVX2_FN static void dequant_row_q4k_avx2(float* dst, const uint8_t* src, size_t n) {
  const __m128i m0f = _mm_set1_epi8(0x0F);
  for (size_t bi = 0; bi < n / 256; bi++) {
    size_t base = bi * 144;
    float d = f16_at(src + base);
    float dmin = f16_at(src + base + 2);
    const uint8_t* scales = src + base + 4;
    const uint8_t* qs = src + base + 16;
    float* out = dst + bi * 256;
    for (int g = 0; g < 4; g++) {
      uint8_t sc1, m1, sc2, m2;
      get_scale_min_k4(2 * g, scales, &sc1, &m1);
      get_scale_min_k4(2 * g + 1, scales, &sc2, &m2);
      __m256 d1 = _mm256_set1_ps(d * (float)sc1), mm1 = _mm256_set1_ps(dmin * (float)m1);
      __m256 d2 = _mm256_set1_ps(d * (float)sc2), mm2 = _mm256_set1_ps(dmin * (float)m2);
      const uint8_t* qsg = qs + g * 32;
      float* olo = out + g * 64;
      float* ohi = out + g * 64 + 32;
      for (int k = 0; k < 4; k++) {
        __m128i b = _mm_loadl_epi64((const __m128i*)(qsg + k * 8));
        __m256 lo = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_and_si128(b, m0f)));
        __m256 hi = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_and_si128(_mm_srli_epi16(b, 4), m0f)));
        _mm256_storeu_ps(olo + k * 8, _mm256_sub_ps(_mm256_mul_ps(lo, d1), mm1));
        _mm256_storeu_ps(ohi + k * 8, _mm256_sub_ps(_mm256_mul_ps(hi, d2), mm2));
      }
    }
  }
}

// simd.rs:963-969
bool split_dequant(uint32_t ty, const uint8_t* src, size_t n, float* dst) {
  if (!simd_available() || ty != ORC_Q4_K || n % 256 != 0) return false;
  dequant_row_q4k_avx2(dst, src, n);
  return true;
}

void quantize_q8(const float* x, size_t n, int8_t* qs, float* scales, int32_t* sums, int32_t* sums16) {
  if (simd_available())  // simd.rs:104-112
    quantize_q8_avx2(x, n, qs, scales, sums, sums16);
  else
    quantize_q8_scalar(x, n, qs, scales, sums, sums16);
}

// Per-block exact integer partial dots (what the float combines consume).
int block_dots(uint32_t ty, const uint8_t* src, size_t n, const int8_t* a, int32_t* out) {
  switch (ty) {
    case ORC_Q4_K:
      for (size_t bi = 0; bi < n / 256; bi++) {
        const uint8_t* qs = src + bi * 144 + 16;
        for (int g = 0; g < 4; g++) {
          int32_t i1 = 0, i2 = 0;
          const int8_t* a1 = a + (bi * 8 + 2 * g) * 32;
          const int8_t* a2 = a1 + 32;
          for (int l = 0; l < 32; l++) {
            i1 += (int32_t)(qs[g * 32 + l] & 0x0F) * a1[l];
            i2 += (int32_t)(qs[g * 32 + l] >> 4) * a2[l];
          }
          out[bi * 8 + 2 * g] = i1;
          out[bi * 8 + 2 * g + 1] = i2;
        }
      }
      return 0;
    case ORC_Q6_K:
      for (size_t bi = 0; bi < n / 256; bi++) {
        const uint8_t* blk = src + bi * 210;
        for (int half = 0; half < 2; half++) {
          const uint8_t* ql = blk + half * 64;
          const uint8_t* qh = blk + 128 + half * 32;
          for (int c = 0; c < 4; c++) {
            for (int sub = 0; sub < 2; sub++) {
              int32_t ss = 0;
              const int8_t* ap = a + (bi * 8 + half * 4 + c) * 32 + sub * 16;
              for (int l = 0; l < 16; l++) {
                int li = sub * 16 + l;
                uint8_t lo = (c & 1) ? ql[32 + li] : ql[li];
                uint8_t nib = (c < 2) ? (lo & 0x0F) : (lo >> 4);
                uint8_t hb = (qh[li] >> (2 * c)) & 3;
                ss += (int32_t)(nib | (hb << 4)) * ap[l];
              }
              out[((bi * 8 + half * 4 + c) * 2) + sub] = ss;
            }
          }
        }
      }
      return 0;
    case ORC_Q8_0:
      for (size_t bi = 0; bi < n / 32; bi++) {
        const int8_t* w = (const int8_t*)(src + bi * 34 + 2);
        int32_t s = 0;
        for (int l = 0; l < 32; l++) s += (int32_t)w[l] * a[bi * 32 + l];
        out[bi] = s;
      }
      return 0;
    case ORC_Q4_0:
      for (size_t bi = 0; bi < n / 32; bi++) {
        const uint8_t* qs = src + bi * 18 + 2;
        int32_t s = 0;
        for (int l = 0; l < 16; l++) {
          s += (int32_t)(qs[l] & 0x0F) * a[bi * 32 + l];
          s += (int32_t)(qs[l] >> 4) * a[bi * 32 + 16 + l];
        }
        out[bi] = s;
      }
      return 0;
    default:
      return -1;
  }
}

}  // namespace orc
