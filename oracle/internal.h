// oracle/internal.h — shared internals of the CPU oracle (test infrastructure).
#pragma once
#include <cstddef>
#include <cstdint>
#include <functional>

namespace orc {

// Borrowed view of a Q8Row (simd.rs:88-101).
struct Q8View {
  const int8_t* qs;
  const float* scales;
  const int32_t* sums;
  const int32_t* sums16;
};

bool simd_available();
float f16_to_f32(uint16_t h);
float f16_to_f32_scalar(uint16_t h);
void get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m);
int block_size(uint32_t ty);
int type_size(uint32_t ty);
void dequant_row(uint32_t ty, const uint8_t* src, size_t n, float* dst);
float dequant_dot_scalar(uint32_t ty, const uint8_t* src, const float* x, size_t n);
bool dequant_dot_avx2(uint32_t ty, const uint8_t* src, const float* x, size_t n, float* out);
void quantize_q8_avx2(const float* x, size_t n, int8_t* qs, float* scales, int32_t* sums, int32_t* sums16);
void quantize_q8_scalar(const float* x, size_t n, int8_t* qs, float* scales, int32_t* sums, int32_t* sums16);
void quantize_q8(const float* x, size_t n, int8_t* qs, float* scales, int32_t* sums, int32_t* sums16);
bool dot_qk_q8_row(uint32_t ty, const uint8_t* src, size_t n, const Q8View& act, float* out);
int block_dots(uint32_t ty, const uint8_t* src, size_t n, const int8_t* a, int32_t* out);
void rmsnorm_core(float* out, const float* x, const float* w, size_t n, float eps);
float dot_f32_avx2(const float* a, const float* b, size_t n);
void saxpy_avx2(float* dst, float alpha, const float* x, size_t n);
void dot_multi(const float* buf, size_t cols, const float* xs, size_t xs_off, size_t xs_stride, size_t n,
               float* out, size_t out_stride);
void dot_multi_rows_3_4(const float* bufs, size_t cols, const float* xs, size_t n, size_t cnt, float* out,
                        size_t out_stride);
bool split_dequant(uint32_t ty, const uint8_t* src, size_t n, float* dst);

// ops.rs
float dot(const float* a, const float* b, size_t n);
float dot_scalar(const float* a, const float* b, size_t n);
void saxpy(float* dst, float alpha, const float* x, size_t n);
void rmsnorm(float* out, const float* x, const float* w, size_t n, float eps, int mode);
void rmsnorm_head(float* p, const float* w, size_t n, float eps, int mode);
float silu(float x);
void softmax_inplace(float* x, size_t n);
void rope_neox_freqs(float* buf, size_t n_heads, size_t head_dim, size_t pos, const float* inv_freq);
void matmul(uint32_t ty, const uint8_t* w, size_t rows, size_t cols, const float* x, float* y, int mode);
void matmul_batch(uint32_t ty, const uint8_t* w, size_t rows, size_t cols, const float* xs, size_t n,
                  float* ys, int mode);

// Fork-join pool standing in for rayon's global pool: each index is handed
// to exactly one worker, so results never depend on the thread count.
void parallel_for(size_t n, const std::function<void(size_t)>& fn);
int num_threads();
void set_num_threads(int n);

}  // namespace orc
