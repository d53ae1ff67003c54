// oracle/capi.cpp — extern "C" entry points of the CPU oracle for ctypes.
// TEST INFRASTRUCTURE ONLY.
#include <vector>

#include "cpu_ref.h"
#include "internal.h"

using namespace orc;

extern "C" {

int orc_type_block_size(uint32_t ty) { return block_size(ty); }
int orc_type_size(uint32_t ty) { return type_size(ty); }
float orc_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
float orc_f16_to_f32_scalar(uint16_t h) { return orc::f16_to_f32_scalar(h); }
void orc_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) { get_scale_min_k4(j, q, sc, m); }

int orc_dequant_row(uint32_t ty, const uint8_t* src, size_t n, float* dst) {
  int bs = block_size(ty);
  if (bs == 0 || n % (size_t)bs != 0) return -1;
  dequant_row(ty, src, n, dst);
  return 0;
}
float orc_dequant_dot_scalar(uint32_t ty, const uint8_t* src, const float* x, size_t n) {
  return dequant_dot_scalar(ty, src, x, n);
}
float orc_dequant_dot(uint32_t ty, const uint8_t* src, const float* x, size_t n) {
  float v;
  if (dequant_dot_avx2(ty, src, x, n, &v)) return v;
  return dequant_dot_scalar(ty, src, x, n);
}

int orc_simd_available(void) { return simd_available() ? 1 : 0; }

void orc_quantize_q8(const float* x, size_t n, int mode, int8_t* qs, float* scales, int32_t* sums,
                     int32_t* sums16) {
  if (mode == 1 || (mode == 0 && simd_available()))
    quantize_q8_avx2(x, n, qs, scales, sums, sums16);
  else
    quantize_q8_scalar(x, n, qs, scales, sums, sums16);
}

int orc_dot_qk_q8_row(uint32_t ty, const uint8_t* src, size_t n, const int8_t* qs, const float* scales,
                      const int32_t* sums, const int32_t* sums16, float* out) {
  Q8View act{qs, scales, sums, sums16};
  return dot_qk_q8_row(ty, src, n, act, out) ? 0 : -1;
}

int orc_block_dots(uint32_t ty, const uint8_t* src, size_t n, const int8_t* qs, int32_t* out) {
  return block_dots(ty, src, n, qs, out);
}

void orc_rmsnorm_avx2(float* out, const float* x, const float* w, size_t n, float eps) {
  rmsnorm_core(out, x, w, n, eps);
}
float orc_dot_f32_avx2(const float* a, const float* b, size_t n) { return dot_f32_avx2(a, b, n); }
void orc_saxpy_avx2(float* dst, float alpha, const float* x, size_t n) { saxpy_avx2(dst, alpha, x, n); }
void orc_dot_multi(const float* buf, size_t cols, const float* xs, size_t xs_off, size_t xs_stride, size_t n,
                   float* out, size_t out_stride) {
  dot_multi(buf, cols, xs, xs_off, xs_stride, n, out, out_stride);
}
void orc_dot_multi_rows_3_4(const float* bufs, size_t cols, const float* xs, size_t n, size_t cnt, float* out,
                            size_t out_stride) {
  dot_multi_rows_3_4(bufs, cols, xs, n, cnt, out, out_stride);
}
int orc_split_dequant(uint32_t ty, const uint8_t* src, size_t n, float* dst) {
  return split_dequant(ty, src, n, dst) ? 1 : 0;
}

void orc_set_threads(int n) { set_num_threads(n); }
int orc_get_threads(void) { return num_threads(); }
float orc_dot(const float* a, const float* b, size_t n) { return dot(a, b, n); }
void orc_matmul(uint32_t ty, const uint8_t* w, size_t rows, size_t cols, const float* x, float* y, int mode) {
  matmul(ty, w, rows, cols, x, y, mode);
}
void orc_matmul_batch(uint32_t ty, const uint8_t* w, size_t rows, size_t cols, const float* xs, size_t n, float* ys,
                      int mode) {
  matmul_batch(ty, w, rows, cols, xs, n, ys, mode);
}
void orc_rmsnorm(float* out, const float* x, const float* w, size_t n, float eps, int mode) {
  rmsnorm(out, x, w, n, eps, mode);
}
void orc_rmsnorm_head(float* p, const float* w, size_t n, float eps, int mode) { rmsnorm_head(p, w, n, eps, mode); }
float orc_silu(float x) { return silu(x); }
void orc_softmax_inplace(float* x, size_t n) { softmax_inplace(x, n); }
void orc_rope_neox_freqs(float* buf, size_t n_heads, size_t head_dim, size_t pos, const float* inv_freq) {
  rope_neox_freqs(buf, n_heads, head_dim, pos, inv_freq);
}

}  // extern "C"
