// oracle/ops.cpp — restatement of src/ops.rs plus a fork-join pool in place of
// rayon. TEST INFRASTRUCTURE ONLY (the parity oracle / CPU baseline).
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

#include "cpu_ref.h"
#include "internal.h"

namespace orc {

// ---------------------------------------------------------------------------
// Fork-join pool. parallel_for(n, fn) runs fn(i) for i in [0, n) across the
// workers and the caller, then returns. Indices are claimed from an atomic
// counter; each index runs on exactly one thread.
// ---------------------------------------------------------------------------
namespace {
struct Pool {
  std::vector<std::thread> workers;
  std::mutex mu;
  std::condition_variable cv_start, cv_done;
  const std::function<void(size_t)>* job = nullptr;
  size_t job_n = 0;
  std::atomic<size_t> next{0};
  size_t generation = 0;
  int active = 0;
  bool stop = false;
  int nthreads = 1;

  void worker_loop() {
    size_t seen = 0;
    for (;;) {
      const std::function<void(size_t)>* fn;
      size_t n;
      {
        std::unique_lock<std::mutex> lk(mu);
        cv_start.wait(lk, [&] { return stop || generation != seen; });
        if (stop) return;
        seen = generation;
        fn = job;
        n = job_n;
      }
      for (size_t i = next.fetch_add(1); i < n; i = next.fetch_add(1)) (*fn)(i);
      {
        std::lock_guard<std::mutex> lk(mu);
        if (--active == 0) cv_done.notify_all();
      }
    }
  }
  void resize(int n) {
    shutdown();
    stop = false;
    nthreads = n < 1 ? 1 : n;
    for (int i = 1; i < nthreads; i++) workers.emplace_back([this] { worker_loop(); });
  }
  void shutdown() {
    {
      std::lock_guard<std::mutex> lk(mu);
      stop = true;
    }
    cv_start.notify_all();
    for (auto& t : workers) t.join();
    workers.clear();
  }
  void run(size_t n, const std::function<void(size_t)>& fn) {
    if (n == 0) return;
    if (workers.empty() || n == 1) {
      for (size_t i = 0; i < n; i++) fn(i);
      return;
    }
    {
      std::lock_guard<std::mutex> lk(mu);
      job = &fn;
      job_n = n;
      next.store(0);
      active = (int)workers.size();
      generation++;
    }
    cv_start.notify_all();
    for (size_t i = next.fetch_add(1); i < n; i = next.fetch_add(1)) fn(i);
    std::unique_lock<std::mutex> lk(mu);
    cv_done.wait(lk, [&] { return active == 0; });
  }
  ~Pool() { shutdown(); }
};
Pool& pool() {
  static Pool* p = [] {
    Pool* q = new Pool();
    unsigned hc = std::thread::hardware_concurrency();
    q->resize(hc ? (int)hc : 1);
    return q;
  }();
  return *p;
}
}  // namespace

void parallel_for(size_t n, const std::function<void(size_t)>& fn) { pool().run(n, fn); }
int num_threads() { return pool().nthreads; }
void set_num_threads(int n) { pool().resize(n); }

static inline bool use_simd(int mode) { return simd_available() && !(mode & ORC_MODE_NO_SIMD); }
static inline bool int_type(uint32_t ty) {
  return ty == ORC_Q4_K || ty == ORC_Q6_K || ty == ORC_Q4_0 || ty == ORC_Q8_0;
}

// ops.rs:21-40
float dot_scalar(const float* a, const float* b, size_t n) {
  float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
  size_t chunks = n / 4;
  for (size_t i = 0; i < chunks; i++) {
    size_t j = i * 4;
    acc0 += a[j] * b[j];
    acc1 += a[j + 1] * b[j + 1];
    acc2 += a[j + 2] * b[j + 2];
    acc3 += a[j + 3] * b[j + 3];
  }
  float acc = (acc0 + acc1) + (acc2 + acc3);
  for (size_t i = chunks * 4; i < n; i++) acc += a[i] * b[i];
  return acc;
}

// ops.rs:9-18
float dot(const float* a, const float* b, size_t n) {
  if (simd_available()) return dot_f32_avx2(a, b, n);
  return dot_scalar(a, b, n);
}
static float dot_m(const float* a, const float* b, size_t n, int mode) {
  return use_simd(mode) ? dot_f32_avx2(a, b, n) : dot_scalar(a, b, n);
}

// ops.rs:318-333
void saxpy(float* dst, float alpha, const float* x, size_t n) {
  if (simd_available()) {
    saxpy_avx2(dst, alpha, x, n);
    return;
  }
  for (size_t i = 0; i < n; i++) dst[i] += alpha * x[i];
}

// ops.rs:336-362
void rmsnorm(float* out, const float* x, const float* w, size_t n, float eps, int mode) {
  if (use_simd(mode)) {
    rmsnorm_core(out, x, w, n, eps);
    return;
  }
  float ss = 0.f;
  for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
  float scale = 1.0f / std::sqrt(ss / (float)n + eps);
  for (size_t i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

// ops.rs:365-390
void rmsnorm_head(float* p, const float* w, size_t n, float eps, int mode) {
  if (use_simd(mode)) {
    rmsnorm_core(p, p, w, n, eps);
    return;
  }
  float ss = 0.f;
  for (size_t i = 0; i < n; i++) ss += p[i] * p[i];
  float scale = 1.0f / std::sqrt(ss / (float)n + eps);
  for (size_t i = 0; i < n; i++) p[i] = p[i] * scale * w[i];
}

// ops.rs:393-395 (f32::exp is glibc expf)
float silu(float x) { return x / (1.0f + std::exp(-x)); }

// ops.rs:398-419
void softmax_inplace(float* x, size_t n) {
  if (n == 0) return;
  float mx = x[0];
  for (size_t i = 1; i < n; i++)
    if (x[i] > mx) mx = x[i];
  float sum = 0.f;
  for (size_t i = 0; i < n; i++) {
    x[i] = std::exp(x[i] - mx);
    sum += x[i];
  }
  if (sum > 0.0f) {
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) x[i] *= inv;
  }
}

// ops.rs:426-446 (f32::sin_cos = glibc sinf, cosf)
void rope_neox_freqs(float* buf, size_t n_heads, size_t head_dim, size_t pos, const float* inv_freq) {
  size_t half = head_dim / 2;
  float p = (float)pos;
  for (size_t h = 0; h < n_heads; h++) {
    float* head = buf + h * head_dim;
    for (size_t i = 0; i < half; i++) {
      float a = p * inv_freq[i];
      float s = std::sin(a), c = std::cos(a);
      float x0 = head[i], x1 = head[i + half];
      head[i] = x0 * c - x1 * s;
      head[i + half] = x0 * s + x1 * c;
    }
  }
}

// ops.rs:67-141
void matmul(uint32_t ty, const uint8_t* w, size_t rows, size_t cols, const float* x, float* y, int mode) {
  if (rows == 0) return;
  size_t rb = (size_t)type_size(ty) * (cols / (size_t)block_size(ty));
  if (ty == ORC_F32) {  // ops.rs:77-83
    const float* ws = (const float*)w;
    parallel_for(rows, [&](size_t r) { y[r] = dot_m(ws + r * cols, x, cols, mode); });
    return;
  }
  size_t nt = (size_t)num_threads();
  size_t chunk = rows / (nt * 4);
  if (chunk < 1) chunk = 1;
  size_t nchunks = (rows + chunk - 1) / chunk;
  if (int_type(ty) && !(mode & ORC_MODE_NO_INT) && use_simd(mode)) {  // ops.rs:93-128
    size_t nb = cols / 32;
    std::vector<int8_t> qs(nb * 32);
    std::vector<float> sc(nb);
    std::vector<int32_t> sums(nb), sums16(nb * 2);
    quantize_q8(x, cols, qs.data(), sc.data(), sums.data(), sums16.data());
    Q8View act{qs.data(), sc.data(), sums.data(), sums16.data()};
    parallel_for(nchunks, [&](size_t ci) {
      size_t base = ci * chunk, end = base + chunk < rows ? base + chunk : rows;
      for (size_t r = base; r < end; r++) dot_qk_q8_row(ty, w + r * rb, cols, act, &y[r]);
    });
    return;
  }
  bool simd = use_simd(mode);  // ops.rs:131-140
  parallel_for(nchunks, [&](size_t ci) {
    size_t base = ci * chunk, end = base + chunk < rows ? base + chunk : rows;
    for (size_t r = base; r < end; r++) {
      float v;
      if (!(simd && dequant_dot_avx2(ty, w + r * rb, x, cols, &v))) v = dequant_dot_scalar(ty, w + r * rb, x, cols);
      y[r] = v;
    }
  });
}

// ops.rs:150-313
void matmul_batch(uint32_t ty, const uint8_t* w, size_t rows, size_t cols, const float* xs, size_t n, float* ys,
                  int mode) {
  if (rows == 0 || n == 0) return;
  if (n == 1) {
    matmul(ty, w, rows, cols, xs, ys, mode);
    return;
  }
  std::memset(ys, 0, sizeof(float) * n * rows);
  if (ty == ORC_F32) {  // ops.rs:167-175
    const float* ws = (const float*)w;
    parallel_for(n, [&](size_t k) {
      for (size_t r = 0; r < rows; r++) ys[k * rows + r] = dot_m(ws + r * cols, xs + k * cols, cols, mode);
    });
    return;
  }
  size_t rb = (size_t)type_size(ty) * (cols / (size_t)block_size(ty));
  size_t nt = (size_t)num_threads();
  size_t chunk = rows / (nt * 4);
  if (chunk < 1) chunk = 1;
  size_t nchunks = (rows + chunk - 1) / chunk;
  bool simd = use_simd(mode);
  if (int_type(ty) && (mode & ORC_MODE_BATCH_INT) && !(mode & ORC_MODE_NO_INT) && simd) {  // ops.rs:192-236
    size_t nb = cols / 32;
    std::vector<int8_t> qs(n * nb * 32);
    std::vector<float> sc(n * nb);
    std::vector<int32_t> sums(n * nb), sums16(n * nb * 2);
    for (size_t k = 0; k < n; k++)
      quantize_q8(xs + k * cols, cols, qs.data() + k * nb * 32, sc.data() + k * nb, sums.data() + k * nb,
                  sums16.data() + k * nb * 2);
    parallel_for(nchunks, [&](size_t ci) {
      size_t base = ci * chunk, end = base + chunk < rows ? base + chunk : rows;
      for (size_t r = base; r < end; r++) {
        for (size_t k = 0; k < n; k++) {
          Q8View act{qs.data() + k * nb * 32, sc.data() + k * nb, sums.data() + k * nb, sums16.data() + k * nb * 2};
          dot_qk_q8_row(ty, w + r * rb, cols, act, &ys[k * rows + r]);
        }
      }
    });
    return;
  }
  constexpr size_t RBLK = 3;  // ops.rs:252-253
  parallel_for(nchunks, [&](size_t ci) {
    size_t base = ci * chunk, end = base + chunk < rows ? base + chunk : rows;
    std::vector<float> buf(cols * RBLK, 0.f);
    size_t r = base;
    while (r < end) {
      size_t cnt = end - r < RBLK ? end - r : RBLK;
      for (size_t j = 0; j < cnt; j++) {
        const uint8_t* row = w + (r + j) * rb;
        bool fast = simd && split_dequant(ty, row, cols, buf.data() + j * cols);
        if (!fast) dequant_row(ty, row, cols, buf.data() + j * cols);
      }
      if (simd) {
        dot_multi_rows_3_4(buf.data(), cols, xs, n, cnt, ys + r, rows);
        r += cnt;
        continue;
      }
      for (size_t j = 0; j < cnt; j++)
        for (size_t k = 0; k < n; k++) ys[k * rows + r + j] = dot_scalar(buf.data() + j * cols, xs + k * cols, cols);
      r += cnt;
    }
  });
}

}  // namespace orc
