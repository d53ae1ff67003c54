// synth.cpp — block quantizers and the seeded synthetic-weight generator.
//
// The reference ships dequantizers only (src/quant.rs:191-385); GGUF files
// it reads were quantized elsewhere. These quantizers are this project's own
// simple encoders for the same block layouts, so a synthetic model can be
// written in any ggml type the hot path reads. Any valid encoding is fine:
// the GPU path and the CPU reference consume the identical bytes.
//
// Synthetic weights: splitmix64 keyed by (seed, tensor id), Box-Muller in
// f64, stored as f32, then quantized row by row.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/rlh.h"

namespace {

uint16_t f32_to_f16(float f) {  // IEEE round-to-nearest-even
  uint32_t x;
  std::memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t mant = x & 0x7fffffu;
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    mant |= 0x800000u;
    int shift = 14 - e;
    uint32_t half = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1);
    uint32_t mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (half & 1))) half++;
    return (uint16_t)(sign | half);
  }
  uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
  return (uint16_t)(sign | h);
}

float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000) << 16, exp = (h >> 10) & 0x1f, mant = h & 0x3ff, bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      uint32_t e = 113;
      while (!(mant & 0x400)) {
        mant <<= 1;
        e--;
      }
      bits = sign | (e << 23) | ((mant & 0x3ff) << 13);
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (mant << 13);
  } else {
    bits = sign | ((exp + 112) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

void put_f16(uint8_t* p, float v) {
  uint16_t h = f32_to_f16(v);
  p[0] = (uint8_t)(h & 0xff);
  p[1] = (uint8_t)(h >> 8);
}

int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

void quant_q8_0(const float* x, size_t n, uint8_t* out) {
  for (size_t b = 0; b < n / 32; b++) {
    const float* xb = x + b * 32;
    uint8_t* o = out + b * 34;
    float amax = 0.f;
    for (int i = 0; i < 32; i++) amax = std::fmax(amax, std::fabs(xb[i]));
    put_f16(o, amax / 127.f);
    float d = f16_to_f32((uint16_t)(o[0] | (o[1] << 8)));
    float id = d > 0.f ? 1.f / d : 0.f;
    for (int i = 0; i < 32; i++) o[2 + i] = (uint8_t)(int8_t)clampi((int)std::lrint(xb[i] * id), -127, 127);
  }
}

void quant_q4_0(const float* x, size_t n, uint8_t* out) {
  for (size_t b = 0; b < n / 32; b++) {
    const float* xb = x + b * 32;
    uint8_t* o = out + b * 18;
    float amax = 0.f;
    for (int i = 0; i < 32; i++) amax = std::fmax(amax, std::fabs(xb[i]));
    put_f16(o, amax / 7.f);
    float d = f16_to_f32((uint16_t)(o[0] | (o[1] << 8)));
    float id = d > 0.f ? 1.f / d : 0.f;
    for (int j = 0; j < 16; j++) {
      int q0 = clampi((int)std::lrint(xb[j] * id) + 8, 0, 15);
      int q1 = clampi((int)std::lrint(xb[j + 16] * id) + 8, 0, 15);
      o[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
  }
}

// Q4_1 / Q5_1: q = round((x - m) / d) with the stored f16 d and m; Q5_0:
// q = round(x / d) + 16. The fifth bit of value t of a block is bit t of the
// block's little-endian qh word (quant.rs Q5_0/Q5_1 arms).
float f16_round(float v) { return f16_to_f32(f32_to_f16(v)); }

template <int BITS, bool MIN>
void quant_q_lin(const float* x, size_t n, uint8_t* out) {
  constexpr int qmax = (1 << BITS) - 1;
  constexpr size_t ts = 2 + (MIN ? 2 : 0) + (BITS == 5 ? 4 : 0) + 16;
  for (size_t b = 0; b < n / 32; b++) {
    const float* xb = x + b * 32;
    uint8_t* o = out + b * ts;
    float lo = xb[0], hi = xb[0], amax = 0.f;
    for (int i = 0; i < 32; i++) {
      lo = std::fmin(lo, xb[i]);
      hi = std::fmax(hi, xb[i]);
      amax = std::fmax(amax, std::fabs(xb[i]));
    }
    const float dv = MIN ? (hi - lo) / (float)qmax : amax / (float)(qmax / 2);
    put_f16(o, dv);
    const float d = f16_round(dv), id = d > 0.f ? 1.f / d : 0.f;
    const float m = MIN ? f16_round(lo) : 0.f;
    if (MIN) put_f16(o + 2, lo);
    uint8_t* qs = o + ts - 16;
    uint32_t qh = 0;
    int q[32];
    for (int i = 0; i < 32; i++) {
      const int v = MIN ? (int)std::lrint((xb[i] - m) * id) : (int)std::lrint(xb[i] * id) + (qmax + 1) / 2;
      q[i] = clampi(v, 0, qmax);
      if (BITS == 5) qh |= (uint32_t)(q[i] >> 4) << i;
    }
    for (int j = 0; j < 16; j++) qs[j] = (uint8_t)((q[j] & 15) | ((q[j + 16] & 15) << 4));
    if (BITS == 5) std::memcpy(o + ts - 20, &qh, 4);
  }
}

// BF16: the upper half of the f32 bits, rounded to nearest even.
void put_bf16(uint8_t* p, float v) {
  uint32_t x;
  std::memcpy(&x, &v, 4);
  const uint16_t h = (x & 0x7fffffffu) > 0x7f800000u ? (uint16_t)((x >> 16) | 0x40u)
                                                      : (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
  p[0] = (uint8_t)(h & 0xff);
  p[1] = (uint8_t)(h >> 8);
}

// Q4_K: 8 sub-blocks of 32 with a 6-bit scale and a 6-bit min each, packed as
// get_scale_min_k4 (quant.rs:176-185) unpacks them.
void quant_q4_k(const float* x, size_t n, uint8_t* out) {
  for (size_t b = 0; b < n / 256; b++) {
    const float* xb = x + b * 256;
    uint8_t* o = out + b * 144;
    float scale[8], mins[8];
    float max_scale = 0.f, max_min = 0.f;
    for (int j = 0; j < 8; j++) {
      float mn = xb[32 * j], mx = xb[32 * j];
      for (int i = 1; i < 32; i++) {
        mn = std::fmin(mn, xb[32 * j + i]);
        mx = std::fmax(mx, xb[32 * j + i]);
      }
      if (mn > 0.f) mn = 0.f;
      scale[j] = (mx - mn) / 15.f;
      mins[j] = -mn;
      max_scale = std::fmax(max_scale, scale[j]);
      max_min = std::fmax(max_min, mins[j]);
    }
    put_f16(o, max_scale / 63.f);
    put_f16(o + 2, max_min / 63.f);
    float d = f16_to_f32((uint16_t)(o[0] | (o[1] << 8)));
    float dmin = f16_to_f32((uint16_t)(o[2] | (o[3] << 8)));
    uint8_t sc[8], m[8];
    for (int j = 0; j < 8; j++) {
      sc[j] = (uint8_t)(d > 0.f ? clampi((int)std::lrint(scale[j] / d), 0, 63) : 0);
      m[j] = (uint8_t)(dmin > 0.f ? clampi((int)std::lrint(mins[j] / dmin), 0, 63) : 0);
    }
    uint8_t* s = o + 4;
    for (int j = 0; j < 4; j++) {
      s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
      s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
      s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
    }
    uint8_t q[256];
    for (int j = 0; j < 8; j++) {
      float dj = d * (float)sc[j], mj = dmin * (float)m[j];
      for (int i = 0; i < 32; i++) {
        int v = dj > 0.f ? (int)std::lrint((xb[32 * j + i] + mj) / dj) : 0;
        q[32 * j + i] = (uint8_t)clampi(v, 0, 15);
      }
    }
    uint8_t* qs = o + 16;
    for (int g = 0; g < 4; g++)
      for (int l = 0; l < 32; l++) qs[32 * g + l] = (uint8_t)(q[64 * g + l] | (q[64 * g + 32 + l] << 4));
  }
}

// Q5_K: as Q4_K with 5-bit quants; the fifth bit of value l of sub-block j
// is bit j of qh[l] (quant.rs:313-349 reads it back).
void quant_q5_k(const float* x, size_t n, uint8_t* out) {
  for (size_t b = 0; b < n / 256; b++) {
    const float* xb = x + b * 256;
    uint8_t* o = out + b * 176;
    float scale[8], mins[8];
    float max_scale = 0.f, max_min = 0.f;
    for (int j = 0; j < 8; j++) {
      float mn = xb[32 * j], mx = xb[32 * j];
      for (int i = 1; i < 32; i++) {
        mn = std::fmin(mn, xb[32 * j + i]);
        mx = std::fmax(mx, xb[32 * j + i]);
      }
      if (mn > 0.f) mn = 0.f;
      scale[j] = (mx - mn) / 31.f;
      mins[j] = -mn;
      max_scale = std::fmax(max_scale, scale[j]);
      max_min = std::fmax(max_min, mins[j]);
    }
    put_f16(o, max_scale / 63.f);
    put_f16(o + 2, max_min / 63.f);
    float d = f16_to_f32((uint16_t)(o[0] | (o[1] << 8)));
    float dmin = f16_to_f32((uint16_t)(o[2] | (o[3] << 8)));
    uint8_t sc[8], m[8];
    for (int j = 0; j < 8; j++) {
      sc[j] = (uint8_t)(d > 0.f ? clampi((int)std::lrint(scale[j] / d), 0, 63) : 0);
      m[j] = (uint8_t)(dmin > 0.f ? clampi((int)std::lrint(mins[j] / dmin), 0, 63) : 0);
    }
    uint8_t* s = o + 4;
    for (int j = 0; j < 4; j++) {
      s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
      s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
      s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
    }
    uint8_t q[256];
    for (int j = 0; j < 8; j++) {
      float dj = d * (float)sc[j], mj = dmin * (float)m[j];
      for (int i = 0; i < 32; i++) {
        int v = dj > 0.f ? (int)std::lrint((xb[32 * j + i] + mj) / dj) : 0;
        q[32 * j + i] = (uint8_t)clampi(v, 0, 31);
      }
    }
    uint8_t* qh = o + 16;
    uint8_t* qs = o + 48;
    for (int l = 0; l < 32; l++) {
      uint8_t h = 0;
      for (int j = 0; j < 8; j++) h |= (uint8_t)(((q[32 * j + l] >> 4) & 1) << j);
      qh[l] = h;
    }
    for (int g = 0; g < 4; g++)
      for (int l = 0; l < 32; l++) qs[32 * g + l] = (uint8_t)((q[64 * g + l] & 15) | ((q[64 * g + 32 + l] & 15) << 4));
  }
}

// Q6_K: 16 sub-blocks of 16 with a signed 8-bit scale each.
void quant_q6_k(const float* x, size_t n, uint8_t* out) {
  for (size_t b = 0; b < n / 256; b++) {
    const float* xb = x + b * 256;
    uint8_t* o = out + b * 210;
    float scale[16], max_abs_scale = 0.f;
    for (int j = 0; j < 16; j++) {
      float amax = 0.f;
      for (int i = 0; i < 16; i++) amax = std::fmax(amax, std::fabs(xb[16 * j + i]));
      scale[j] = amax / 31.f;
      max_abs_scale = std::fmax(max_abs_scale, scale[j]);
    }
    put_f16(o + 208, max_abs_scale / 127.f);
    float d = f16_to_f32((uint16_t)(o[208] | (o[209] << 8)));
    int8_t sc[16];
    for (int j = 0; j < 16; j++) sc[j] = (int8_t)(d > 0.f ? clampi((int)std::lrint(scale[j] / d), -128, 127) : 0);
    uint8_t u[256];
    for (int j = 0; j < 16; j++) {
      float dj = d * (float)sc[j];
      for (int i = 0; i < 16; i++) {
        int v = dj != 0.f ? (int)std::lrint(xb[16 * j + i] / dj) : 0;
        u[16 * j + i] = (uint8_t)(clampi(v, -32, 31) + 32);
      }
    }
    uint8_t* ql = o;
    uint8_t* qh = o + 128;
    for (int h = 0; h < 2; h++) {
      for (int l = 0; l < 32; l++) {
        uint8_t u1 = u[128 * h + l], u2 = u[128 * h + l + 32], u3 = u[128 * h + l + 64], u4 = u[128 * h + l + 96];
        ql[64 * h + l] = (uint8_t)((u1 & 0xF) | ((u3 & 0xF) << 4));
        ql[64 * h + l + 32] = (uint8_t)((u2 & 0xF) | ((u4 & 0xF) << 4));
        qh[32 * h + l] = (uint8_t)((u1 >> 4) | ((u2 >> 4) << 2) | ((u3 >> 4) << 4) | ((u4 >> 4) << 6));
      }
    }
    std::memcpy(o + 192, sc, 16);
  }
}

inline uint64_t splitmix64_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}
constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ULL;

// Value i of the N(mean, std) stream of (seed, tensor id): element pairs
// (2p, 2p+1) come from one Box-Muller draw on uniforms p*2+1, p*2+2.
void normal_stream(uint64_t seed, uint64_t tensor_id, uint64_t offset, uint64_t n, float mean, float stdv,
                   float* out) {
  uint64_t key = splitmix64_mix(seed + kGamma * (tensor_id + 1));
  const double two_pi = 6.283185307179586476925286766559;
  uint64_t i = offset, end = offset + n;
  while (i < end) {
    uint64_t p = i / 2;
    uint64_t a = splitmix64_mix(key + kGamma * (2 * p + 1));
    uint64_t bb = splitmix64_mix(key + kGamma * (2 * p + 2));
    double u1 = (double)((a >> 11) + 1) * (1.0 / 9007199254740992.0);  // (0, 1]
    double u2 = (double)(bb >> 11) * (1.0 / 9007199254740992.0);       // [0, 1)
    double r = std::sqrt(-2.0 * std::log(u1));
    double s = std::sin(two_pi * u2), c = std::cos(two_pi * u2);
    if ((i & 1) == 0) {
      out[i - offset] = (float)(mean + stdv * r * c);
      i++;
      if (i < end) {
        out[i - offset] = (float)(mean + stdv * r * s);
        i++;
      }
    } else {
      out[i - offset] = (float)(mean + stdv * r * s);
      i++;
    }
  }
}

}  // namespace

extern "C" {

int rlh_quantize_row(uint32_t ty, const float* src, uint64_t n, void* dst) {
  uint8_t* o = (uint8_t*)dst;
  switch (ty) {
    case RLH_TYPE_F32: std::memcpy(o, src, n * 4); return 0;
    case RLH_TYPE_F16:
      for (uint64_t i = 0; i < n; i++) put_f16(o + 2 * i, src[i]);
      return 0;
    case RLH_TYPE_BF16:
      for (uint64_t i = 0; i < n; i++) put_bf16(o + 2 * i, src[i]);
      return 0;
    case RLH_TYPE_Q4_1: if (n % 32) return -1; quant_q_lin<4, true>(src, n, o); return 0;
    case RLH_TYPE_Q5_0: if (n % 32) return -1; quant_q_lin<5, false>(src, n, o); return 0;
    case RLH_TYPE_Q5_1: if (n % 32) return -1; quant_q_lin<5, true>(src, n, o); return 0;
    case RLH_TYPE_Q8_0: if (n % 32) return -1; quant_q8_0(src, n, o); return 0;
    case RLH_TYPE_Q4_0: if (n % 32) return -1; quant_q4_0(src, n, o); return 0;
    case RLH_TYPE_Q4_K: if (n % 256) return -1; quant_q4_k(src, n, o); return 0;
    case RLH_TYPE_Q5_K: if (n % 256) return -1; quant_q5_k(src, n, o); return 0;
    case RLH_TYPE_Q6_K: if (n % 256) return -1; quant_q6_k(src, n, o); return 0;
    default: return -2;
  }
}

void rlh_synth_normal(uint64_t seed, uint64_t tensor_id, uint64_t offset, uint64_t n, float mean, float stdv,
                      float* out) {
  normal_stream(seed, tensor_id, offset, n, mean, stdv, out);
}

int rlh_synth_tensor(uint64_t seed, uint64_t tensor_id, uint32_t ty, uint64_t rows, uint64_t cols, float mean,
                     float stdv, void* dst, int nthreads) {
  uint64_t rb = rlh_row_bytes(ty, cols);
  if (rb == 0) return -1;
  if (nthreads < 1) nthreads = 1;
  std::vector<std::thread> th;
  std::vector<int> err(nthreads, 0);
  for (int t = 0; t < nthreads; t++) {
    th.emplace_back([&, t] {
      std::vector<float> buf(cols);
      for (uint64_t r = t; r < rows; r += nthreads) {
        normal_stream(seed, tensor_id, r * cols, cols, mean, stdv, buf.data());
        if (rlh_quantize_row(ty, buf.data(), cols, (uint8_t*)dst + r * rb) != 0) err[t] = 1;
      }
    });
  }
  for (auto& x : th) x.join();
  for (int e : err)
    if (e) return -2;
  return 0;
}

void rlh_synth_tokens(uint64_t seed, uint64_t n, uint32_t vocab, uint32_t* out) {
  uint64_t key = splitmix64_mix(seed ^ 0x70726f6d7074ULL);  // "prompt"
  for (uint64_t i = 0; i < n; i++) out[i] = (uint32_t)(splitmix64_mix(key + kGamma * (i + 1)) % vocab);
}

}  // extern "C"
