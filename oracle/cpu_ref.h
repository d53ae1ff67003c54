// oracle/cpu_ref.h — CPU restatement of rust-llama's Qwen3 token loop.
//
// TEST INFRASTRUCTURE ONLY. This code is the parity oracle and the CPU
// baseline. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
// leg may load it, and only to check results against. The product path (librlh.so)
// never links or calls anything here.
//
// It restates, function by function, the reference's x86-64 AVX2 path
// (the production path on any AVX2+FMA+F16C host) plus the portable scalar
// fallbacks, with the same intrinsic names as Rust's std::arch::x86_64:
//   src/quant.rs   block formats, f16, get_scale_min_k4, dequant_row,
//                  dequant_dot_scalar
//   src/simd.rs    quantize_q8 (AVX2 + scalar), integer Q x Q8 dots,
//                  fused f32 dequant-dots, rmsnorm_core, dot_f32, saxpy,
//                  dot_multi(_rows), split dequant of Q4_K
//   src/ops.rs     matmul / matmul_batch dispatch, rmsnorm(_head), silu,
//                  softmax_inplace, rope_neox_freqs
//   src/model.rs   Config, KvCache, forward_one / forward_batch /
//                  forward_into, generate
//   src/sampler.rs Sampler (xorshift64*), greedy fast path
//   src/main.rs    argmax and the bench protocol
// Compiled with -ffp-contract=off: Rust never contracts a*b+c into an FMA, so
// every FMA below is an explicit _mm256_fmadd_ps exactly where the reference
// has one.
//
// Parity status per function (how each is pinned is in tests/):
//   dequant, f16, scale unpack, integer block dots, quantize_q8: pinned by
//     closed forms (independent numpy restatement of the block formats),
//     brute-force integer identities and the reference's own invariants.
//   float combines, rmsnorm, dot_f32, saxpy, dot_multi_rows: pinned by the
//     reference's own self-consistency tests (simd.rs:1097-1484, ops.rs:478-573)
//     and by f64 closed forms.
//   forward_one / forward_batch op order: pinned against an independent f64
//     numpy forward of a small model.
//   sampler: pinned by the reference's own tests (sampler.rs:181-206) plus
//     the xorshift64* closed form.
//   libm calls (expf, sinf, cosf, powf): glibc of the host image, as the
//     reference links it; parity of glibc itself is not pinned here.
#pragma once
#include <cstddef>
#include <cstdint>

extern "C" {

// ggml type ids (quant.rs:26-41)
enum {
  ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q5_0 = 6, ORC_Q5_1 = 7,
  ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_BF16 = 30
};

// --- block formats / quant.rs ---------------------------------------------
int orc_type_block_size(uint32_t ty);                // quant.rs:44-50 (0 if unknown)
int orc_type_size(uint32_t ty);                      // quant.rs:53-66
float orc_f16_to_f32(uint16_t h);                    // quant.rs:115-123 (F16C when available)
float orc_f16_to_f32_scalar(uint16_t h);             // quant.rs:134-157
void orc_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m);  // quant.rs:176-185
int orc_dequant_row(uint32_t ty, const uint8_t* src, size_t n, float* dst);   // quant.rs:191-385
float orc_dequant_dot_scalar(uint32_t ty, const uint8_t* src, const float* x, size_t n);  // quant.rs:409-541
// quant.rs:392-400: AVX2 kernel when the type has one (simd.rs:38-51), else scalar.
float orc_dequant_dot(uint32_t ty, const uint8_t* src, const float* x, size_t n);

// --- simd.rs ----------------------------------------------------------------
int orc_simd_available(void);                        // simd.rs:17-34 (also honours ORC_NO_SIMD)
// Q8Row (simd.rs:88-101): qs[n], scales[n/32], sums[n/32], sums16[n/16]
// mode 0 = quantize_q8 dispatch (AVX2 if available), 1 = AVX2, 2 = scalar.
void orc_quantize_q8(const float* x, size_t n, int mode, int8_t* qs, float* scales,
                     int32_t* sums, int32_t* sums16);
// Integer dot of one row against a Q8Row (simd.rs:898-910). Returns 0 and
// writes *out on success, -1 when the type has no integer kernel.
int orc_dot_qk_q8_row(uint32_t ty, const uint8_t* src, size_t n, const int8_t* qs,
                      const float* scales, const int32_t* sums, const int32_t* sums16,
                      float* out);
// Exact integer partial dots the float combine consumes:
//   Q4_K: per 32-value block, sum(nibble * a)           -> n/32 values
//   Q6_K: per 16-value half-block, sum(u * a), u=q+32   -> n/16 values
//   Q8_0: per 32-value block, sum(w * a)                -> n/32 values
//   Q4_0: per 32-value block, sum(nibble * a)           -> n/32 values
int orc_block_dots(uint32_t ty, const uint8_t* src, size_t n, const int8_t* qs, int32_t* out);
void orc_rmsnorm_avx2(float* out, const float* x, const float* w, size_t n, float eps);  // simd.rs:282-326
float orc_dot_f32_avx2(const float* a, const float* b, size_t n);                       // simd.rs:328-377
void orc_saxpy_avx2(float* dst, float alpha, const float* x, size_t n);                 // simd.rs:674-691
void orc_dot_multi(const float* buf, size_t cols, const float* xs, size_t xs_off,
                   size_t xs_stride, size_t n, float* out, size_t out_stride);           // simd.rs:700-754
void orc_dot_multi_rows_3_4(const float* bufs, size_t cols, const float* xs, size_t n,
                            size_t cnt, float* out, size_t out_stride);                  // simd.rs:782-836
int orc_split_dequant(uint32_t ty, const uint8_t* src, size_t n, float* dst);          // simd.rs:963-969

// --- ops.rs -------------------------------------------------------------------
// Execution modes mirror the reference's env toggles.
enum { ORC_MODE_DEFAULT = 0, ORC_MODE_NO_INT = 1, ORC_MODE_BATCH_INT = 2, ORC_MODE_NO_SIMD = 4 };
// Not a reference mode: decode attention with its softmax and PV sums taken
// over four position splits (the summation order of a split-K kernel), for
// tests that measure how far a reordered f32 sum moves the greedy sequence.
enum { ORC_MODE_SPLIT_ATTN = 8 };
void orc_set_threads(int n);
int orc_get_threads(void);
float orc_dot(const float* a, const float* b, size_t n);                                // ops.rs:9-18
void orc_matmul(uint32_t ty, const uint8_t* w, size_t rows, size_t cols, const float* x,
                float* y, int mode);                                                     // ops.rs:67-141
void orc_matmul_batch(uint32_t ty, const uint8_t* w, size_t rows, size_t cols,
                      const float* xs, size_t n, float* ys, int mode);                   // ops.rs:150-313
void orc_rmsnorm(float* out, const float* x, const float* w, size_t n, float eps, int mode);  // ops.rs:336-362
void orc_rmsnorm_head(float* p, const float* w, size_t n, float eps, int mode);         // ops.rs:365-390
float orc_silu(float x);                                                                 // ops.rs:393-395
void orc_softmax_inplace(float* x, size_t n);                                            // ops.rs:398-419
void orc_rope_neox_freqs(float* buf, size_t n_heads, size_t head_dim, size_t pos,
                         const float* inv_freq);                                         // ops.rs:426-446

// --- model.rs -------------------------------------------------------------------
typedef struct orc_config {      // model.rs:15-29
  uint32_t n_layer, n_embd, n_ff, n_head, n_head_kv, head_dim;
  float rope_theta, rms_eps;
  uint32_t n_ctx, vocab_size;
  uint32_t has_qk_norm, has_output;
} orc_config;

// Tensor kinds: GGUF names blk.{l}.<kind>.weight / token_embd / output(_norm).
enum {
  ORC_T_TOKEN_EMBD = 0, ORC_T_OUTPUT_NORM = 1, ORC_T_OUTPUT = 2,
  ORC_T_ATTN_NORM = 3, ORC_T_ATTN_Q = 4, ORC_T_ATTN_K = 5, ORC_T_ATTN_V = 6,
  ORC_T_ATTN_OUTPUT = 7, ORC_T_ATTN_Q_NORM = 8, ORC_T_ATTN_K_NORM = 9,
  ORC_T_FFN_NORM = 10, ORC_T_FFN_GATE = 11, ORC_T_FFN_UP = 12, ORC_T_FFN_DOWN = 13,
  ORC_T_ATTN_Q_BIAS = 14, ORC_T_ATTN_K_BIAS = 15, ORC_T_ATTN_V_BIAS = 16
};

typedef struct orc_model orc_model;
typedef struct orc_cache orc_cache;
orc_model* orc_model_create(const orc_config* cfg);
// Borrows `bytes` (the caller keeps them alive for the model's lifetime),
// as Model borrows the mmap (model.rs:331-337). Norms/biases are converted
// to f32 at set time, as Model::load does (model.rs:156-162).
int orc_model_set_tensor(orc_model* m, int kind, int layer, uint32_t ty, const void* bytes,
                         size_t n_cols, size_t n_rows);
int orc_model_finalize(orc_model* m);
void orc_model_destroy(orc_model* m);
orc_cache* orc_cache_create(orc_model* m, size_t max_ctx);      // model.rs:339-342 (clamped)
void orc_cache_reset(orc_cache* c);                             // model.rs:131-133
size_t orc_cache_len(const orc_cache* c);
size_t orc_cache_max_ctx(const orc_cache* c);
void orc_cache_destroy(orc_cache* c);
// model.rs:353-375; `mode` selects the ops.rs toggles for this call.
void orc_forward_into(orc_model* m, orc_cache* c, const uint32_t* tokens, size_t n,
                      size_t start_pos, float* logits, int mode);
// When set, forward passes copy the residual stream after every layer into
// `buf` (layout [n_layer][n_tokens][n_embd]); pass NULL to disable.
void orc_set_hidden_dump(orc_cache* c, float* buf, size_t max_tokens);
// K/V cache rows of one layer (f32 [max_ctx][kv_dim]) for parity checks.
const float* orc_cache_k(const orc_cache* c, int layer);
const float* orc_cache_v(const orc_cache* c, int layer);

// --- sampler.rs / main.rs ---------------------------------------------------------
typedef struct orc_sampling_params {     // sampler.rs:3-26
  float temperature;
  uint32_t top_k;
  float top_p;
  float repetition_penalty;
  uint32_t repeat_last_n;
  uint64_t seed;
} orc_sampling_params;
typedef struct orc_sampler orc_sampler;
orc_sampler* orc_sampler_create(uint64_t seed);                 // sampler.rs:33-37
void orc_sampler_destroy(orc_sampler* s);
uint64_t orc_sampler_next_u64(orc_sampler* s);                  // sampler.rs:40-48
float orc_sampler_next_f32(orc_sampler* s);                     // sampler.rs:51-54
uint32_t orc_sampler_sample(orc_sampler* s, const float* logits, size_t n,
                            const orc_sampling_params* p, const uint32_t* recent,
                            size_t n_recent);                   // sampler.rs:56-163
uint32_t orc_argmax(const float* x, size_t n);                  // main.rs:453-463
// model.rs:741-776 (EOS handling: stops when `eos` is produced; pass
// 0xFFFFFFFF to ignore EOS as the bench protocol here does).
size_t orc_generate(orc_model* m, orc_cache* c, const uint32_t* prompt, size_t n_prompt,
                    size_t max_new, const orc_sampling_params* p, uint32_t eos,
                    uint32_t* out_tokens, int mode);

// The bench protocol of main.rs:466-530: warm-up prefill, reset, timed prefill,
// timed greedy decode loop (argmax after every step). EOS is ignored.
typedef struct orc_bench_result {
  double prefill_s, decode_s;
  size_t prompt_len, generated;
} orc_bench_result;
int orc_bench(orc_model* m, orc_cache* c, const uint32_t* prompt, size_t n_prompt,
              size_t n_gen, int mode, int do_warmup, orc_bench_result* out, uint32_t* out_tokens);

}  // extern "C"
