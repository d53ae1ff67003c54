/* rlh.h — C ABI of the MI355X (gfx950) Qwen3 token loop.
 *
 * This is the drop-in boundary behind the reference's Rust API. A Rust host
 * keeps `Model::forward_into` / `KvCache` / the sampler and binds these
 * symbols through a thin FFI crate (an `extern "C"` block that mirrors
 * every declaration below one to one).
 * Plain C types only: pointers, sizes and status codes; no torch or HIP
 * types cross the boundary.
 *
 * Conventions
 *  - Every entry returning `int` returns RLH_OK (0) on success and a negative
 *    RLH_E* code on failure; `rlh_last_error()` then describes the failure
 *    (thread-local). Nothing here aborts on bad input: shape, type and
 *    context errors are reported, where the reference would `assert!`
 *    (src/ops.rs:70-71, 153-154).
 *  - Host pointers (`const void* host_bytes`, `float* logits`, ...) are
 *    borrowed for the duration of the call only.
 *  - A model is immutable after rlh_model_finalize and may be shared by
 *    several caches. A cache owns one HIP stream and its device KV memory;
 *    calls on one cache must be serialised by the caller, as the reference
 *    requires `&mut KvCache` (src/model.rs:353-359; server.rs:5-10).
 *  - Numerics follow the reference's AVX2 production path bit for bit:
 *    decode (`rlh_forward_one`) and batched prefill (`rlh_forward_batch`,
 *    integer semantics of RUST_LLAMA_BATCH_INT=1, src/ops.rs:192-236) return
 *    the same f32 logits, K/V rows and hidden states as that path.
 */
#ifndef RLH_H
#define RLH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define RLH_OK 0
#define RLH_EINVAL (-1)   /* bad argument, shape or type                      */
#define RLH_ENOMEM (-2)   /* device or host allocation failed                 */
#define RLH_EDEVICE (-3)  /* HIP runtime error                                */
#define RLH_ESTATE (-4)   /* wrong call order (e.g. model not finalized)      */
#define RLH_ECTX (-5)     /* position at or beyond the cache's max_ctx        */
#define RLH_EUNSUP (-6)   /* valid ggml type with no kernel on this path      */
#define RLH_EIO (-7)      /* file cannot be opened, mapped or written         */
#define RLH_EFORMAT (-8)  /* malformed GGUF file or missing metadata          */
#define RLH_ENOENT (-9)   /* no such metadata key or tensor                   */

/* ---- ggml tensor types (src/quant.rs:26-41, ids as in GGUF) ----------- */
#define RLH_TYPE_F32 0u
#define RLH_TYPE_F16 1u
#define RLH_TYPE_Q4_0 2u
#define RLH_TYPE_Q4_1 3u
#define RLH_TYPE_Q5_0 6u
#define RLH_TYPE_Q5_1 7u
#define RLH_TYPE_Q8_0 8u
#define RLH_TYPE_Q4_K 12u
#define RLH_TYPE_Q5_K 13u
#define RLH_TYPE_Q6_K 14u
#define RLH_TYPE_BF16 30u

/* ---- tensor kinds (GGUF names resolved by Model::load, src/model.rs:164-218) */
#define RLH_T_TOKEN_EMBD 0   /* token_embd.weight                   */
#define RLH_T_OUTPUT_NORM 1  /* output_norm.weight                  */
#define RLH_T_OUTPUT 2       /* output.weight (absent when tied)    */
#define RLH_T_ATTN_NORM 3    /* blk.{l}.attn_norm.weight            */
#define RLH_T_ATTN_Q 4       /* blk.{l}.attn_q.weight               */
#define RLH_T_ATTN_K 5       /* blk.{l}.attn_k.weight               */
#define RLH_T_ATTN_V 6       /* blk.{l}.attn_v.weight               */
#define RLH_T_ATTN_OUTPUT 7  /* blk.{l}.attn_output.weight          */
#define RLH_T_ATTN_Q_NORM 8  /* blk.{l}.attn_q_norm.weight          */
#define RLH_T_ATTN_K_NORM 9  /* blk.{l}.attn_k_norm.weight          */
#define RLH_T_FFN_NORM 10    /* blk.{l}.ffn_norm.weight             */
#define RLH_T_FFN_GATE 11    /* blk.{l}.ffn_gate.weight             */
#define RLH_T_FFN_UP 12      /* blk.{l}.ffn_up.weight               */
#define RLH_T_FFN_DOWN 13    /* blk.{l}.ffn_down.weight             */
#define RLH_T_ATTN_Q_BIAS 14 /* blk.{l}.attn_q.bias (Qwen2 only)    */
#define RLH_T_ATTN_K_BIAS 15 /* blk.{l}.attn_k.bias                 */
#define RLH_T_ATTN_V_BIAS 16 /* blk.{l}.attn_v.bias                 */

/* Model hyper-parameters: the fields of `Config` (src/model.rs:15-29). */
typedef struct rlh_config {
  uint32_t n_layer, n_embd, n_ff, n_head, n_head_kv, head_dim;
  float rope_theta, rms_eps;
  uint32_t n_ctx, vocab_size;
  uint32_t has_qk_norm, has_output;
} rlh_config;

typedef struct rlh_model rlh_model;
typedef struct rlh_cache rlh_cache;

/* Description of the last failure on this thread ("" if none). */
const char* rlh_last_error(void);
/* Library version string. */
const char* rlh_version(void);

/* Bytes of one row of `cols` elements (GgmlType::row_size, quant.rs:69-73);
 * 0 for an unknown type or a length that is not a whole number of blocks. */
uint64_t rlh_row_bytes(uint32_t ggml_type, uint64_t cols);

/* ---- model ---------------------------------------------------------------
 * Replaces Model::load (src/model.rs:150-239): the caller resolves tensors
 * (from GGUF or a generator) and hands them over one by one. */
/* Whether this path runs a model of this config, without a device: RLH_OK,
 * RLH_EINVAL (zero dimensions, n_head not a multiple of n_head_kv) or
 * RLH_EUNSUP with the reason (head_dim other than 128, n_embd or n_ff not a
 * multiple of 256, more than 8 query heads per KV head). The reference's
 * read_config (src/model.rs:241-293) accepts these shapes; rlh_model_create
 * and rlh_model_load_gguf apply this check before anything is uploaded. */
int rlh_config_check(const rlh_config* cfg);
int rlh_model_create(const rlh_config* cfg, rlh_model** out);
/* Copies one tensor to device memory (the host bytes are borrowed only for
 * the call, as Tensor borrows the mmap, src/tensor.rs:6-35). Norm and bias
 * vectors are converted to f32 as Model::load does (model.rs:156-162).
 * `layer` is ignored for the global kinds. n_cols = elements per row. */
int rlh_model_set_tensor(rlh_model* m, int kind, int layer, uint32_t ggml_type, const void* host_bytes,
                         uint64_t n_cols, uint64_t n_rows);
/* Validates that every tensor the forward pass needs is present with
 * consistent shapes (the arch gate and "missing tensor" errors of
 * model.rs:41-52, 794-808), builds the RoPE tables and freezes the model. */
int rlh_model_finalize(rlh_model* m);
void rlh_model_destroy(rlh_model* m);
/* Device bytes held by the model's weights. */
uint64_t rlh_model_weight_bytes(const rlh_model* m);

/* ---- GGUF files -------------------------------------------------------------
 * The reference's GGUF v2/v3 reader (GgufFile, src/gguf.rs:125-421): the
 * file is memory-mapped, metadata parsed eagerly, tensor bytes borrowed from
 * the mapping while the handle is open. Malformed files (bad magic, other
 * versions, truncation, absurd counts or lengths, unknown value or tensor
 * types) return RLH_EFORMAT without aborting (gguf.rs:433-464). */
typedef struct rlh_gguf rlh_gguf;
/* GgufFile::open (gguf.rs:246-307), including the sibling files of a split
 * model (split.count > 1, named "-0000k-of-0000n.gguf" as gguf.rs:262-273). */
int rlh_gguf_open(const char* path, rlh_gguf** out);
void rlh_gguf_close(rlh_gguf* g);
uint32_t rlh_gguf_version(const rlh_gguf* g);
/* Files mapped (1 + the split siblings found). */
uint64_t rlh_gguf_n_files(const rlh_gguf* g);
/* Tensors in file order (tensor_order, gguf.rs:127) and their TensorInfo
 * (gguf.rs:90-123): name, ggml type, dims (dims[0] = row length; up to
 * max_dims written, *n_dims = all), offset in its file's data section, file. */
uint64_t rlh_gguf_n_tensors(const rlh_gguf* g);
int rlh_gguf_tensor_info(const rlh_gguf* g, uint64_t index, const char** name, uint32_t* ggml_type,
                         uint32_t* n_dims, uint64_t* dims, uint32_t max_dims, uint64_t* offset,
                         uint32_t* file_index);
/* GgufFile::tensor_bytes (gguf.rs:385-413): the tensor's bytes inside the
 * mapping (valid until rlh_gguf_close); RLH_ENOENT for an unknown name,
 * RLH_EFORMAT when they extend past the end of the file. */
int rlh_gguf_tensor_bytes(const rlh_gguf* g, const char* name, const void** data, uint64_t* nbytes);
/* Metadata: keys in file order; value type (GGUF value type ids 0-12, the
 * element type and count of an array); MetaValue::as_u32 / as_f32 /
 * as_str (gguf.rs:32-88) and raw scalars (u: unsigned and bool, i: signed,
 * f: float). A missing key returns RLH_ENOENT, a value of another type
 * RLH_EINVAL. Strings stay valid until rlh_gguf_close. */
uint64_t rlh_gguf_n_meta(const rlh_gguf* g);
int rlh_gguf_meta_key(const rlh_gguf* g, uint64_t index, const char** key);
int rlh_gguf_meta_type(const rlh_gguf* g, const char* key, uint32_t* type, uint32_t* elem_type, uint64_t* n_elems);
int rlh_gguf_meta_u32(const rlh_gguf* g, const char* key, uint32_t* v);
int rlh_gguf_meta_f32(const rlh_gguf* g, const char* key, float* v);
int rlh_gguf_meta_scalar(const rlh_gguf* g, const char* key, uint64_t* u, int64_t* i, double* f);
int rlh_gguf_meta_str(const rlh_gguf* g, const char* key, const char** s, uint64_t* len);
int rlh_gguf_meta_arr_str(const rlh_gguf* g, const char* key, uint64_t index, const char** s, uint64_t* len);
int rlh_gguf_meta_arr_scalar(const rlh_gguf* g, const char* key, uint64_t index, uint64_t* u, int64_t* i,
                             double* f);
/* Model::read_config (model.rs:241-293): general.architecture (default
 * "llama", copied to `arch`) must be qwen3 or qwen2 (check_arch,
 * model.rs:794-808, RLH_EUNSUP otherwise); each key is read as
 * "{arch}.{key}", then as "{key}", with the reference's defaults. */
int rlh_gguf_config(const rlh_gguf* g, rlh_config* cfg, char* arch, uint64_t arch_cap);
/* Model::load (model.rs:150-239): the config, the vocabulary check of
 * read_tokenizer (tokenizer.ggml.tokens, model.rs:295-300), then every
 * tensor by its GGUF name through rlh_model_set_tensor, and finalize. The
 * GGUF may be closed afterwards (the device holds its own copies). */
int rlh_model_load_gguf(const rlh_gguf* g, rlh_model** out);

/* GGUF writer (write_gguf, src/prune.rs:381-442): metadata written in key
 * byte order, tensors in the order added with their data offsets aligned to
 * `alignment`, the data section aligned. Tensor bytes are borrowed until
 * rlh_gguf_writer_write. Value types are the GGUF ids; a string array takes
 * `values` as an array of NUL-terminated strings, a numeric array packed
 * little-endian values; arrays of arrays are refused. */
typedef struct rlh_gguf_writer rlh_gguf_writer;
int rlh_gguf_writer_create(uint32_t version, uint64_t alignment, rlh_gguf_writer** out);
void rlh_gguf_writer_destroy(rlh_gguf_writer* w);
int rlh_gguf_writer_set_scalar(rlh_gguf_writer* w, const char* key, uint32_t type, const void* value);
int rlh_gguf_writer_set_string(rlh_gguf_writer* w, const char* key, const char* s, uint64_t len);
int rlh_gguf_writer_set_array(rlh_gguf_writer* w, const char* key, uint32_t elem_type, const void* values, uint64_t n);
int rlh_gguf_writer_add_tensor(rlh_gguf_writer* w, const char* name, uint32_t ggml_type, uint32_t n_dims,
                               const uint64_t* dims, const void* data, uint64_t nbytes);
int rlh_gguf_writer_write(rlh_gguf_writer* w, const char* path);

/* Vocabulary pruning (prune::prune_vocab, src/prune.rs:127-291): rewrites
 * in_path (split files included) to out_path keeping every unknown,
 * control, user-defined and byte token, every token a *_token_id key names,
 * and the tokens whose text has no character of the dropped scripts (the
 * reference's table of ranges: Cyrillic, CJK, Indic, ...); the rows of
 * token_embd / output that have one row per token, the merges whose parts
 * and result survive, and every *_token_id value remapped (as u32). All
 * other metadata and tensors are copied. RLH_EFORMAT ("prune: ...") for a
 * missing vocabulary, a token_type array of another length, an empty result
 * or a named token that was dropped. `stats` (nullable) receives the counts
 * of PruneStats. */
typedef struct rlh_prune_stats {
  uint64_t old_vocab, new_vocab, kept_special, kept_byte, kept_normal, dropped;
  uint64_t merges_old, merges_new, embd_bytes_saved, out_bytes;
} rlh_prune_stats;
int rlh_prune_vocab(const char* in_path, const char* out_path, rlh_prune_stats* stats);

/* ---- tokenizer and chat template ---------------------------------------------
 * The reference's byte-level BPE tokenizer (GPT-2 / Qwen2 flavour,
 * src/tokenizer.rs): GPT-2 byte-to-unicode mapping, the Qwen2 pre-tokenizer
 * pattern written out with Rust's char::is_alphabetic / is_numeric /
 * is_whitespace, merges applied lowest rank first (leftmost on equal rank),
 * token types 3 and 4 matched verbatim as special tokens (longest first). */
typedef struct rlh_tokenizer rlh_tokenizer;
/* Tokenizer::new (tokenizer.rs:56-112): tokens (NUL-terminated), their types
 * (1 for entries past n_types), merges "left right" in rank order. */
int rlh_tokenizer_create(const char* const* tokens, uint64_t n_tokens, const uint32_t* token_types, uint64_t n_types,
                         const char* const* merges, uint64_t n_merges, uint32_t bos_id, uint32_t eos_id,
                         rlh_tokenizer** out);
/* Model::read_tokenizer (model.rs:295-330): tokenizer.ggml.tokens (required),
 * .token_type, .merges, .bos_token_id (default 1), .eos_token_id (default 2). */
int rlh_tokenizer_from_gguf(const rlh_gguf* g, rlh_tokenizer** out);
void rlh_tokenizer_destroy(rlh_tokenizer* t);
uint64_t rlh_tokenizer_vocab_size(const rlh_tokenizer* t);
uint32_t rlh_tokenizer_bos(const rlh_tokenizer* t);
uint32_t rlh_tokenizer_eos(const rlh_tokenizer* t);
/* Tokenizer::encode (tokenizer.rs:299-334) of len bytes of UTF-8 text
 * (RLH_EINVAL if invalid). *n_ids receives the token count; when it exceeds
 * cap the first cap ids are written and RLH_EINVAL is returned. An empty
 * special token string never matches (the reference would loop on it). */
int rlh_tokenizer_encode(const rlh_tokenizer* t, const char* text, uint64_t len, uint32_t* ids, uint64_t cap,
                         uint64_t* n_ids);
/* The pre-tokenizer's pieces (tokenizer.rs:142-246) as byte ranges
 * [bounds[2k], bounds[2k+1]); cap counts uint64 entries (2 per piece). */
int rlh_tokenizer_pretokenize(const rlh_tokenizer* t, const char* text, uint64_t len, uint64_t* bounds, uint64_t cap,
                              uint64_t* n_pieces);
/* Tokenizer::decode (tokenizer.rs:336-359): the ids' bytes as lossy UTF-8
 * (unknown ids skipped). *len receives the byte length; the text is
 * NUL-terminated when it fits; RLH_EINVAL when it exceeds cap. */
int rlh_tokenizer_decode(const rlh_tokenizer* t, const uint32_t* ids, uint64_t n, char* out, uint64_t cap,
                         uint64_t* len);
/* Tokenizer::token_bytes (tokenizer.rs:124-140): the raw bytes of one token. */
int rlh_tokenizer_token_bytes(const rlh_tokenizer* t, uint32_t id, char* out, uint64_t cap, uint64_t* len);
/* format_qwen_multiturn (tokenizer.rs:403-430; with no turns it is
 * format_qwen_chat, 386-401): optional system block, the (role, content)
 * turns, the user prompt, the assistant header and, with no_think, the
 * empty think block. Strings are NUL-terminated; `system` may be NULL. */
int rlh_format_qwen_chat(const char* const* roles, const char* const* contents, uint64_t n_turns, const char* prompt,
                         const char* system, int no_think, char* out, uint64_t cap, uint64_t* len);

/* ---- KV cache ------------------------------------------------------------
 * Replaces Model::new_cache / KvCache (src/model.rs:107-134, 339-342):
 * f32 K and V per layer in the same [pos][kv_head][head_dim] layout.
 * max_ctx is clamped to cfg.n_ctx exactly as model.rs:340 does. */
int rlh_cache_create(rlh_model* m, uint64_t max_ctx, rlh_cache** out);
int rlh_cache_reset(rlh_cache* c); /* KvCache::reset: len = 0, no zeroing */
uint64_t rlh_cache_len(const rlh_cache* c);
uint64_t rlh_cache_max_ctx(const rlh_cache* c);
void rlh_cache_destroy(rlh_cache* c);

/* ---- forward pass ----------------------------------------------------------
 * All three return once `logits` (host, >= vocab_size floats, may be NULL to
 * skip the copy) holds the last token's logits. */
/* Model::forward_one with logits (src/model.rs:585-738): one decode step at
 * `pos`; writes K/V at pos; cache len becomes pos + 1. */
int rlh_forward_one(rlh_model* m, rlh_cache* c, uint32_t token, uint64_t pos, float* logits);
/* Model::forward_batch (src/model.rs:384-583): n tokens from start_pos,
 * truncated to max_ctx - start_pos (model.rs:392); logits of the last one. */
int rlh_forward_batch(rlh_model* m, rlh_cache* c, const uint32_t* tokens, uint64_t n, uint64_t start_pos,
                      float* logits);
/* Model::forward_into (src/model.rs:353-375): n > 1 -> batch, n == 1 -> one. */
int rlh_forward_into(rlh_model* m, rlh_cache* c, const uint32_t* tokens, uint64_t n, uint64_t start_pos,
                     float* logits);
/* Greedy argmax of the logits computed by the last forward call on this
 * cache, on device, with main.rs argmax semantics (main.rs:453-463): the
 * lowest index among equal maxima, NaN never wins, 0 when no value exceeds
 * -inf. (The sampler's greedy fast path, sampler.rs:62-70, differs only in
 * keeping index 0 when logits[0] is NaN; rlh_sample_next applies that.) */
int rlh_greedy_next(rlh_model* m, rlh_cache* c, uint32_t* token);
/* The greedy token loop of cmd_bench (src/main.rs:500-516) run on device:
 * starting from `first` at position cache len, n_steps decode steps, each
 * feeding the argmax of the previous step. out_tokens[i] receives the token
 * fed at step i, out_tokens[n_steps] the argmax after the last step. EOS is
 * not checked (the bench protocol here fixes the token count). Stops early
 * with RLH_ECTX when the cache is full. */
int rlh_generate_greedy(rlh_model* m, rlh_cache* c, uint32_t first, uint64_t n_steps, uint32_t* out_tokens);

/* ---- sampling (src/sampler.rs, src/model.rs:741-776) ----------------------------- */
/* SamplingParams (sampler.rs:3-26); defaults there: 0.7, 40, 0.95, 1.1, 64,
 * 0x123456789abcdef0. */
typedef struct rlh_sampling_params {
  float temperature;        /* <= 0: greedy                                     */
  uint32_t top_k;           /* 0: all tokens                                    */
  float top_p;              /* applied when in (0, 1)                           */
  float repetition_penalty; /* 1: off                                           */
  uint32_t repeat_last_n;   /* window of the penalty; 0: whole history          */
  uint64_t seed;            /* Sampler::new(seed) (used by rlh_generate)        */
} rlh_sampling_params;
/* Sampler::new (sampler.rs:33-37): the xorshift64* state for a seed. */
uint64_t rlh_sampler_init(uint64_t seed);
/* Sampler::sample (sampler.rs:56-163) on host logits[n] with the history
 * `recent`; advances *rng_state. Equal probabilities inside top-k are
 * ordered by token id (the reference leaves their order to Rust's
 * select_nth_unstable). */
int rlh_sample(const float* logits, uint64_t n, const rlh_sampling_params* p, const uint32_t* recent,
               uint64_t n_recent, uint64_t* rng_state, uint32_t* token);
/* ops::softmax_inplace (src/ops.rs:398-419) on host x[n], as the sampler
 * runs it (sampler.rs:119): max, exp(x - max) with the platform expf's
 * results, the sum in index order, then x * (1 / sum) when the sum is > 0. */
int rlh_softmax(float* x, uint64_t n);
/* The same on the logits of the last forward call on this cache, on the
 * device (rlh_dsampler_sample on the cache's stream); only the token comes
 * back to the host. */
int rlh_sample_next(rlh_model* m, rlh_cache* c, const rlh_sampling_params* p, const uint32_t* recent,
                    uint64_t n_recent, uint64_t* rng_state, uint32_t* token);

/* Device sampler: Sampler::sample (src/sampler.rs:56-163) and
 * ops::softmax_inplace (src/ops.rs:398-419) on device-resident values, with
 * the tokens, probabilities and RNG states of rlh_sample / rlh_softmax bit
 * for bit. The reference samples on the host after forward_into copies the
 * logits out (model.rs:353-375, 741-776); these replace that copy and the
 * host pass. A handle holds device workspace for n <= max_n on the device
 * current at creation; calls on one handle must not overlap. */
typedef struct rlh_dsampler rlh_dsampler;
int rlh_dsampler_create(uint64_t max_n, rlh_dsampler** out);
void rlh_dsampler_destroy(rlh_dsampler* ds);
/* logits: device f32[n]. recent, rng_state and token are host memory. The
 * stream (hipStream_t, NULL: the null stream) orders the reads of logits;
 * the call returns after the token is known. Logits that turn into NaN or
 * infinity after the penalty and temperature give RLH_EINVAL (the
 * reference's sort panics on them); the RNG state is then unchanged. */
int rlh_dsampler_sample(rlh_dsampler* ds, const float* logits, uint64_t n, const rlh_sampling_params* p,
                        const uint32_t* recent, uint64_t n_recent, uint64_t* rng_state, uint32_t* token,
                        void* stream);
/* Softmax of device x[n] in place, enqueued on the stream (no wait). */
int rlh_dsampler_softmax(rlh_dsampler* ds, float* x, uint64_t n, void* stream);
/* Largest candidate list the top-k / top-p search sorts on chip (default and
 * maximum 4096); longer lists, and 0 here, take the full radix sort. */
int rlh_dsampler_set_candidate_cap(rlh_dsampler* ds, uint32_t cap);
/* How the last rlh_dsampler_sample call chose its token (RLH_DSAMPLER_PATH_*). */
#define RLH_DSAMPLER_PATH_GREEDY 1u     /* argmax (temperature <= 0)               */
#define RLH_DSAMPLER_PATH_CANDIDATES 2u /* candidate list sorted on chip           */
#define RLH_DSAMPLER_PATH_SORT 4u       /* radix sort of every probability         */
#define RLH_DSAMPLER_PATH_FALLBACK 8u   /* candidates did not fit: sorted instead  */
uint32_t rlh_dsampler_last_path(const rlh_dsampler* ds);
/* Model::generate (src/model.rs:741-776): reset the cache, prefill the
 * prompt (n_prompt >= 1), then up to max_new steps of sample -> stop at
 * `eos` -> append -> stop when the cache is full -> decode. out_tokens
 * (max_new entries) receives the generated tokens, *n_out their count. */
int rlh_generate(rlh_model* m, rlh_cache* c, const uint32_t* prompt, uint64_t n_prompt, uint64_t max_new,
                 const rlh_sampling_params* p, uint32_t eos, uint32_t* out_tokens, uint64_t* n_out);

/* ---- inspection for parity tests --------------------------------------------- */
/* Residual stream after `layer` for the tokens of the last forward call
 * (n_tokens x n_embd f32, token-major). Requires rlh_cache_set_debug(c, 1)
 * before that call. */
int rlh_cache_set_debug(rlh_cache* c, int enable);
int rlh_debug_layer_hidden(rlh_cache* c, int layer, float* out, uint64_t max_tokens);
/* K or V rows [0, n_pos) of one layer: n_pos x (n_head_kv*head_dim) f32. */
int rlh_cache_read_kv(rlh_cache* c, int layer, int which_v, uint64_t n_pos, float* out);

/* ---- op-level entries (host buffers in and out) ----------------------------------
 * Each uploads its inputs, runs the device kernel the forward pass uses and
 * copies results back. */
/* simd::quantize_q8 (src/simd.rs:104-203, AVX2 rounding: ties to even):
 * qs[n], scales[n/32], sums[n/32], sums16[n/16]; n must be a multiple of 32. */
int rlh_quantize_q8(const float* x, uint64_t n, int8_t* qs, float* scales, int32_t* sums, int32_t* sums16);
/* quant::dequant_row (src/quant.rs:191-385) over n elements. */
int rlh_dequant(uint32_t ggml_type, const void* bytes, uint64_t n, float* out);
/* ops::matmul (src/ops.rs:67-141), integer path: y = W x with x quantized
 * to Q8 blocks once. */
int rlh_matvec(uint32_t ggml_type, const void* w, uint64_t rows, uint64_t cols, const float* x, float* y);
/* ops::matmul_batch with RUST_LLAMA_BATCH_INT=1 (src/ops.rs:192-236):
 * ys[k*rows + r] (token-major). */
int rlh_matmul_batch(uint32_t ggml_type, const void* w, uint64_t rows, uint64_t cols, const float* xs, uint64_t n,
                     float* ys);
/* Exact integer partial dots of W against Q8 activation bytes (the values
 * the float combines of simd.rs:581/663/863/891 consume): per row,
 * Q4_K/Q8_0/Q4_0 -> cols/32 values (one per 32-value block),
 * Q6_K -> cols/16 values (one per 16-value half-block, unsigned u = q+32). */
int rlh_block_dots(uint32_t ggml_type, const void* w, uint64_t rows, uint64_t cols, const int8_t* q8, int32_t* out);

/* ---- greedy argmax without allocation -----------------------------------------------
 * The greedy argmax over n floats the caller already holds in device
 * memory, written to the device word *token: the lowest index among equal
 * maxima wins, a NaN never wins, and the token is 0 when no value exceeds
 * -inf. No counterpart in the reference: for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops).
 * Allocates nothing and does not synchronize: the two kernels are enqueued
 * on `stream` (a hipStream_t, NULL for the null stream) and the token is
 * valid once the stream reaches them. Their 256 partial (value, index)
 * pairs live in a 2 KB static device array per GPU, held until the process
 * ends; every call writes all of them before reading, and calls that
 * overlap on one GPU race on them. n must be in [1, 2^32 - 1]; logits and
 * token must be device-accessible memory (RLH_EINVAL otherwise). */
int rlh_argmax_noalloc(const float* logits, uint64_t n, uint32_t* token, void* stream);

/* ---- measurement ---------------------------------------------------------------------
 * Runs the decode launch of one weight kind `iters` times on the cache's
 * stream, rotating over the layers' copies (so weights stream from HBM as in
 * a decode step), and reports the average time per launch in microseconds
 * from one HIP event pair around the back-to-back launches (each launch's
 * dispatch gap included, as inside a captured step). The launch is built as the
 * decode step builds it: RLH_T_ATTN_Q = the fused rmsnorm + q/k/v launch,
 * RLH_T_FFN_GATE / RLH_T_FFN_UP = the fused rmsnorm + gate/up + silu*up
 * launch, other kinds = that matrix alone. No reference counterpart
 * (measurement hook for the bench). */
int rlh_profile_matvec(rlh_model* m, rlh_cache* c, int kind, int iters, double* avg_us);
/* Average duration of one launch of the decode matvec of weight kind `kind`
 * (RLH_T_ATTN_Q = the rmsnorm + q/k/v launch, RLH_T_ATTN_OUTPUT,
 * RLH_T_FFN_GATE = the rmsnorm + gate/up + silu*up launch, RLH_T_FFN_DOWN,
 * RLH_T_OUTPUT = the logits) inside real decode steps: `steps` greedy decode
 * steps starting from token `first` at the cache's length run eagerly, and
 * each launch of that kind takes its own start and end times on the cache's
 * stream (HIP events bound to the launch, hipExtLaunchKernel), the same span
 * a kernel trace reports. *launches receives the number of timed launches;
 * the cache advances by `steps`. No reference counterpart (measurement). */
int rlh_profile_decode_kernel(rlh_model* m, rlh_cache* c, int kind, uint32_t first, int steps, double* avg_us,
                              uint64_t* launches);
/* Average duration of one captured decode step (graph launch) over `iters`
 * steps at the cache's current length, in microseconds; the cache position
 * advances by `iters`. */
int rlh_profile_decode(rlh_model* m, rlh_cache* c, int iters, double* avg_us);

/* ---- synthetic models (host only) ------------------------------------------------------
 * The reference ships no quantizer; these are this project's encoders for
 * the same block layouts, used to write seeded synthetic models. */
int rlh_quantize_row(uint32_t ggml_type, const float* src, uint64_t n, void* dst);
/* Elements [offset, offset+n) of the N(mean, std) stream of (seed, tensor_id). */
void rlh_synth_normal(uint64_t seed, uint64_t tensor_id, uint64_t offset, uint64_t n, float mean, float stdv,
                      float* out);
/* Fills dst (rows * rlh_row_bytes(type, cols) bytes) with a quantized
 * N(mean, std) matrix; row r holds stream elements [r*cols, (r+1)*cols). */
int rlh_synth_tensor(uint64_t seed, uint64_t tensor_id, uint32_t ggml_type, uint64_t rows, uint64_t cols, float mean,
                     float stdv, void* dst, int nthreads);
/* n token ids uniform over [0, vocab). */
void rlh_synth_tokens(uint64_t seed, uint64_t n, uint32_t vocab, uint32_t* out);

#ifdef __cplusplus
}
#endif
#endif /* RLH_H */
