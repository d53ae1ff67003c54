"""ctypes binding of librlh.so (include/rlh.h) plus the synthetic-model specs.

This is the Python stand-in for the thin FFI crate a Rust host would bind
(the reference's `Model::forward_into` / `KvCache` surface, src/model.rs).
It loads the in-tree library and raises if it is missing: there is no CPU
fallback behind it.
"""
import ctypes
import os
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("RLH_LIB") or os.path.join(_HERE, "librlh.so")  # RLH_LIB: another build of the library

# ggml type ids (src/quant.rs:26-41)
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 3, 6, 7, 8, 12, 13, 14, 30
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q4_1: "Q4_1", Q5_0: "Q5_0", Q5_1: "Q5_1", Q8_0: "Q8_0",
              Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", BF16: "BF16"}
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22),
         Q5_1: (32, 24), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}

# tensor kinds (include/rlh.h)
T_TOKEN_EMBD, T_OUTPUT_NORM, T_OUTPUT = 0, 1, 2
T_ATTN_NORM, T_ATTN_Q, T_ATTN_K, T_ATTN_V, T_ATTN_OUTPUT = 3, 4, 5, 6, 7
T_ATTN_Q_NORM, T_ATTN_K_NORM, T_FFN_NORM, T_FFN_GATE, T_FFN_UP, T_FFN_DOWN = 8, 9, 10, 11, 12, 13
T_ATTN_Q_BIAS, T_ATTN_K_BIAS, T_ATTN_V_BIAS = 14, 15, 16
KIND_NAMES = {0: "token_embd", 1: "output_norm", 2: "output", 3: "attn_norm", 4: "attn_q", 5: "attn_k",
              6: "attn_v", 7: "attn_output", 8: "attn_q_norm", 9: "attn_k_norm", 10: "ffn_norm",
              11: "ffn_gate", 12: "ffn_up", 13: "ffn_down", 14: "attn_q_bias", 15: "attn_k_bias",
              16: "attn_v_bias"}

RLH_OK, RLH_EINVAL, RLH_ENOMEM, RLH_EDEVICE, RLH_ESTATE, RLH_ECTX, RLH_EUNSUP = 0, -1, -2, -3, -4, -5, -6
RLH_EIO, RLH_EFORMAT, RLH_ENOENT = -7, -8, -9

# GGUF metadata value types (src/gguf.rs:204-235)
GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32, GGUF_BOOL = 0, 1, 2, 3, 4, 5, 6, 7
GGUF_STR, GGUF_ARR, GGUF_U64, GGUF_I64, GGUF_F64 = 8, 9, 10, 11, 12
_GGUF_NP = {GGUF_U8: np.uint8, GGUF_I8: np.int8, GGUF_U16: np.uint16, GGUF_I16: np.int16, GGUF_U32: np.uint32,
            GGUF_I32: np.int32, GGUF_F32: np.float32, GGUF_BOOL: np.uint8, GGUF_U64: np.uint64,
            GGUF_I64: np.int64, GGUF_F64: np.float64}


def row_bytes(ty, cols):
    bs, ts = BLOCK[ty]
    assert cols % bs == 0
    return cols // bs * ts


class Config(ctypes.Structure):
    """`Config` of src/model.rs:15-29."""
    _fields_ = [("n_layer", ctypes.c_uint32), ("n_embd", ctypes.c_uint32), ("n_ff", ctypes.c_uint32),
                ("n_head", ctypes.c_uint32), ("n_head_kv", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
                ("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float), ("n_ctx", ctypes.c_uint32),
                ("vocab_size", ctypes.c_uint32), ("has_qk_norm", ctypes.c_uint32), ("has_output", ctypes.c_uint32)]


class PruneStats(ctypes.Structure):
    """`PruneStats` of src/prune.rs:113-124."""
    _fields_ = [(f, ctypes.c_uint64) for f in ("old_vocab", "new_vocab", "kept_special", "kept_byte",
                                                "kept_normal", "dropped", "merges_old", "merges_new",
                                                "embd_bytes_saved", "out_bytes")]


@dataclass
class ModelSpec:
    """Shape and per-tensor ggml types of a synthetic Qwen3 model."""
    name: str
    n_layer: int
    n_embd: int
    n_ff: int
    n_head: int
    n_head_kv: int
    vocab: int
    tied: bool
    types: dict = field(default_factory=dict)   # kind -> ggml type
    head_dim: int = 128
    rope_theta: float = 1e6
    rms_eps: float = 1e-6
    n_ctx: int = 40960

    def config(self):
        return Config(self.n_layer, self.n_embd, self.n_ff, self.n_head, self.n_head_kv, self.head_dim,
                      self.rope_theta, self.rms_eps, self.n_ctx, self.vocab, 1, 0 if self.tied else 1)

    def shapes(self):
        """(kind, rows, cols) of every matrix of one layer."""
        E, F, qd, kvd = self.n_embd, self.n_ff, self.n_head * self.head_dim, self.n_head_kv * self.head_dim
        return [(T_ATTN_Q, qd, E), (T_ATTN_K, kvd, E), (T_ATTN_V, kvd, E), (T_ATTN_OUTPUT, E, qd),
                (T_FFN_GATE, F, E), (T_FFN_UP, F, E), (T_FFN_DOWN, E, F)]

    def weight_bytes_per_token(self):
        """Packed bytes of every matrix one decode step reads (7 per layer plus
        the logits matrix) and one embedding row."""
        total = 0
        for kind, rows, cols in self.shapes():
            total += rows * row_bytes(self.types[kind], cols)
        total *= self.n_layer
        out_ty = self.types[T_TOKEN_EMBD] if self.tied else self.types[T_OUTPUT]
        total += self.vocab * row_bytes(out_ty, self.n_embd)
        total += row_bytes(self.types[T_TOKEN_EMBD], self.n_embd)
        return total

    def int8_ops_per_token(self):
        """2 * sum(rows*cols) over the 7 layer matrices (prefill MACs per token)."""
        return 2 * self.n_layer * sum(r * c for _, r, c in self.shapes())


def _q4km(tied, embd_type, out_type):
    t = {T_ATTN_Q: Q4_K, T_ATTN_K: Q4_K, T_ATTN_V: Q6_K, T_ATTN_OUTPUT: Q4_K, T_FFN_GATE: Q4_K,
         T_FFN_UP: Q4_K, T_FFN_DOWN: Q6_K, T_TOKEN_EMBD: embd_type}
    if not tied:
        t[T_OUTPUT] = out_type
    return t


def _q5km():
    """Q5_K_M-like mix: Q5_K everywhere but attn_v / ffn_down in Q6_K; tied Q5_K embedding."""
    return {T_ATTN_Q: Q5_K, T_ATTN_K: Q5_K, T_ATTN_V: Q6_K, T_ATTN_OUTPUT: Q5_K, T_FFN_GATE: Q5_K,
            T_FFN_UP: Q5_K, T_FFN_DOWN: Q6_K, T_TOKEN_EMBD: Q5_K}


def _all(ty, tied=True):
    t = {k: ty for k in (T_ATTN_Q, T_ATTN_K, T_ATTN_V, T_ATTN_OUTPUT, T_FFN_GATE, T_FFN_UP, T_FFN_DOWN,
                         T_TOKEN_EMBD)}
    if not tied:
        t[T_OUTPUT] = ty
    return t


# The five Qwen3 workloads of the benchmark plan plus small shapes for tests.
SPECS = {
    "qwen3-0.6b-q4km": ModelSpec("qwen3-0.6b-q4km", 28, 1024, 3072, 16, 8, 151936, True, _q4km(True, Q4_K, None)),
    "qwen3-0.6b-q8_0": ModelSpec("qwen3-0.6b-q8_0", 28, 1024, 3072, 16, 8, 151936, True, _all(Q8_0)),
    "qwen3-4b-q4km": ModelSpec("qwen3-4b-q4km", 36, 2560, 9728, 32, 8, 151936, True, _q4km(True, Q6_K, None)),
    "qwen3-8b-q4km": ModelSpec("qwen3-8b-q4km", 36, 4096, 12288, 32, 8, 151936, False, _q4km(False, Q4_K, Q6_K)),
    "qwen3-32b-q4km": ModelSpec("qwen3-32b-q4km", 64, 5120, 25600, 64, 8, 151936, False, _q4km(False, Q4_K, Q6_K)),
    # small shapes for parity tests (same code paths, seconds on the CPU oracle)
    "tiny-q4km": ModelSpec("tiny-q4km", 2, 256, 512, 4, 2, 1000, True, _q4km(True, Q4_K, None), n_ctx=512),
    "tiny-q4km-untied": ModelSpec("tiny-q4km-untied", 2, 512, 768, 4, 1, 2048, False, _q4km(False, Q4_K, Q6_K),
                                  n_ctx=512),
    "tiny-q8_0": ModelSpec("tiny-q8_0", 2, 256, 512, 4, 2, 1000, True, _all(Q8_0), n_ctx=512),
    "tiny-q4_0": ModelSpec("tiny-q4_0", 2, 256, 512, 4, 4, 1000, True, _all(Q4_0), n_ctx=512),
    "small-q4km": ModelSpec("small-q4km", 4, 1024, 3072, 16, 8, 4096, False, _q4km(False, Q4_K, Q6_K), n_ctx=1024),
    # Q5_K matrices (no integer path in the reference: f32 products)
    "tiny-q5km": ModelSpec("tiny-q5km", 2, 256, 512, 4, 2, 1000, True, _q5km(), n_ctx=512),
    # the remaining weight types: 32-value blocks with a min and/or a fifth
    # bit (no integer path in the reference) and float rows
    "tiny-q4_1": ModelSpec("tiny-q4_1", 2, 256, 512, 4, 2, 1000, True, _all(Q4_1), n_ctx=512),
    "tiny-q5_0": ModelSpec("tiny-q5_0", 2, 256, 512, 4, 2, 1000, False, _all(Q5_0, tied=False), n_ctx=512),
    "tiny-q5_1": ModelSpec("tiny-q5_1", 2, 256, 512, 4, 2, 1000, True, _all(Q5_1), n_ctx=512),
    "tiny-f16": ModelSpec("tiny-f16", 2, 256, 512, 4, 2, 1000, True, _all(F16), n_ctx=512),
    "tiny-bf16": ModelSpec("tiny-bf16", 2, 256, 512, 4, 2, 1000, False, _all(BF16, tied=False), n_ctx=512),
    "tiny-f32": ModelSpec("tiny-f32", 2, 256, 512, 4, 2, 1000, True, _all(F32), n_ctx=512),
    # one launch mixing float and tiled rows (q/k/v), ffn_gate and ffn_up of
    # different types (separate launches + silu(g)*u), eight types in all
    "tiny-mix": ModelSpec("tiny-mix", 2, 256, 512, 4, 2, 1000, False,
                          {T_ATTN_Q: F16, T_ATTN_K: Q8_0, T_ATTN_V: Q5_1, T_ATTN_OUTPUT: BF16, T_FFN_GATE: Q4_1,
                           T_FFN_UP: Q5_0, T_FFN_DOWN: F32, T_TOKEN_EMBD: Q4_0, T_OUTPUT: Q5_K}, n_ctx=512),
    # f32-product types with a 13056-wide FFN: ffn_down rows too long for the
    # whole-row decode plan (the launch stages the f32 row only and takes a
    # ring plan)
    "tiny-longff-q5": ModelSpec("tiny-longff-q5", 2, 256, 13056, 4, 2, 1000, False,
                                {**_all(Q5_0, tied=False), T_FFN_DOWN: Q5_1, T_FFN_UP: Q4_1, T_FFN_GATE: Q4_1},
                                n_ctx=512),
    # hidden width above both the vocabulary and the FFN width (a small or
    # pruned vocabulary): the cache's f32 temporaries must hold E floats
    "tiny-smallvocab": ModelSpec("tiny-smallvocab", 2, 1024, 512, 8, 4, 300, False, _q4km(False, Q4_K, Q6_K),
                                 n_ctx=512),
    # 8 query heads per KV head (the 32B grouping) and a long context window
    "tiny-g8-q4km": ModelSpec("tiny-g8-q4km", 2, 256, 512, 16, 2, 1000, True, _q4km(True, Q4_K, None), n_ctx=8192),
    # 4 query heads per KV head (the 4B / 8B grouping) and a long context window
    "tiny-g4-q4km": ModelSpec("tiny-g4-q4km", 2, 256, 512, 8, 2, 1000, True, _q4km(True, Q4_K, None), n_ctx=8192),
    # 1 and 2 query heads per KV head with a long context window
    "tiny-g1-q4km": ModelSpec("tiny-g1-q4km", 2, 256, 512, 2, 2, 1000, True, _q4km(True, Q4_K, None), n_ctx=4096),
    "tiny-g2-q4km": ModelSpec("tiny-g2-q4km", 2, 256, 512, 4, 2, 1000, True, _q4km(True, Q4_K, None), n_ctx=4096),
    # groups that do not divide the kernels' 64-wide tiles: 3, 5 (Qwen3-14B's
    # 40/8), 6 and 7 (Qwen2.5-7B's 28/4) query heads per KV head
    "tiny-g3-q4km": ModelSpec("tiny-g3-q4km", 2, 256, 512, 6, 2, 1000, True, _q4km(True, Q4_K, None), n_ctx=4096),
    "tiny-g5-q4km": ModelSpec("tiny-g5-q4km", 2, 256, 512, 10, 2, 1000, True, _q4km(True, Q4_K, None), n_ctx=4096),
    "tiny-g6-q4km": ModelSpec("tiny-g6-q4km", 2, 256, 512, 12, 2, 1000, True, _q4km(True, Q4_K, None), n_ctx=4096),
    "tiny-g7-q4km": ModelSpec("tiny-g7-q4km", 2, 256, 512, 14, 2, 1000, True, _q4km(True, Q4_K, None), n_ctx=4096),
    # 104 query heads (13312-wide attention rows: attn_output takes Q8 blocks
    # from the attention kernels instead of quantizing the row itself)
    "tiny-wide-q4km": ModelSpec("tiny-wide-q4km", 2, 256, 512, 104, 13, 1000, True, _q4km(True, Q4_K, None),
                                n_ctx=4096),
}


# The five benchmark workloads: number -> (model, prompt tokens, decode
# tokens, sampled decode). 4 is the headline. Sampled decode uses the CLI's
# sampling defaults (src/main.rs:44-52): temperature 0.7, top-k 40,
# top-p 0.95, repetition penalty 1.1 over the last 64 tokens, its fixed seed.
WORKLOADS = {
    1: ("qwen3-0.6b-q4km", 48, 32, False),
    2: ("qwen3-0.6b-q8_0", 48, 128, False),
    3: ("qwen3-4b-q4km", 256, 256, False),
    4: ("qwen3-8b-q4km", 512, 512, False),
    5: ("qwen3-32b-q4km", 4096, 256, True),
}
# Seed of the synthetic weights of the workloads; the prompt ids use seed + 1.
WORKLOAD_SEED = 20260


def tensor_id(kind, layer):
    return kind * 4096 + max(layer, 0)


def synth_model(spec, seed, lib=None, nthreads=None):
    """Seeded synthetic weights: N(0, 0.02) matrices quantized by this
    project's encoders, norms 1 + N(0, 0.02) in F32. Returns a list of
    (kind, layer, type, cols, rows, uint8 array)."""
    lib = lib or load()
    nthreads = nthreads or min(16, os.cpu_count() or 1)
    out = []

    def mat(kind, layer, rows, cols, ty):
        buf = np.empty(rows * row_bytes(ty, cols), dtype=np.uint8)
        rc = lib.rlh_synth_tensor(seed, tensor_id(kind, layer), ty, rows, cols, 0.0, 0.02,
                                  buf.ctypes.data, nthreads)
        if rc != 0:
            raise RuntimeError(f"synth tensor {KIND_NAMES[kind]} failed: {rc}")
        out.append((kind, layer, ty, cols, rows, buf))

    def norm(kind, layer, n):
        v = np.empty(n, dtype=np.float32)
        lib.rlh_synth_normal(seed, tensor_id(kind, layer), 0, n, 1.0, 0.02, v.ctypes.data)
        out.append((kind, layer, F32, n, 1, v.view(np.uint8)))

    E = spec.n_embd
    mat(T_TOKEN_EMBD, 0, spec.vocab, E, spec.types[T_TOKEN_EMBD])
    norm(T_OUTPUT_NORM, 0, E)
    if not spec.tied:
        mat(T_OUTPUT, 0, spec.vocab, E, spec.types[T_OUTPUT])
    for l in range(spec.n_layer):
        norm(T_ATTN_NORM, l, E)
        norm(T_FFN_NORM, l, E)
        norm(T_ATTN_Q_NORM, l, spec.head_dim)
        norm(T_ATTN_K_NORM, l, spec.head_dim)
        for kind, rows, cols in spec.shapes():
            mat(kind, l, rows, cols, spec.types[kind])
    return out


def synth_tokens(seed, n, vocab, lib=None):
    lib = lib or load()
    out = np.empty(n, dtype=np.uint32)
    lib.rlh_synth_tokens(seed, n, vocab, out.ctypes.data)
    return out


class SamplingParams(ctypes.Structure):
    """rlh_sampling_params = SamplingParams (src/sampler.rs:3-26)."""
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_uint32), ("top_p", ctypes.c_float),
                ("repetition_penalty", ctypes.c_float), ("repeat_last_n", ctypes.c_uint32),
                ("seed", ctypes.c_uint64)]


def sampling_params(temperature=0.7, top_k=40, top_p=0.95, repetition_penalty=1.1, repeat_last_n=64,
                    seed=0x123456789ABCDEF0):
    """Defaults of SamplingParams::default (sampler.rs:15-26)."""
    return SamplingParams(temperature, top_k, top_p, repetition_penalty, repeat_last_n, seed)


_lib = None


def load():
    """Loads librlh.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
    lib = ctypes.CDLL(LIB_PATH)
    P, U32, U64, I32, F = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int, ctypes.c_float
    sig = {
        "rlh_last_error": (ctypes.c_char_p, []),
        "rlh_version": (ctypes.c_char_p, []),
        "rlh_row_bytes": (U64, [U32, U64]),
        "rlh_config_check": (I32, [ctypes.POINTER(Config)]),
        "rlh_model_create": (I32, [ctypes.POINTER(Config), ctypes.POINTER(P)]),
        "rlh_model_set_tensor": (I32, [P, I32, I32, U32, P, U64, U64]),
        "rlh_model_finalize": (I32, [P]),
        "rlh_model_destroy": (None, [P]),
        "rlh_model_weight_bytes": (U64, [P]),
        "rlh_cache_create": (I32, [P, U64, ctypes.POINTER(P)]),
        "rlh_cache_reset": (I32, [P]),
        "rlh_cache_len": (U64, [P]),
        "rlh_cache_max_ctx": (U64, [P]),
        "rlh_cache_destroy": (None, [P]),
        "rlh_forward_one": (I32, [P, P, U32, U64, P]),
        "rlh_forward_batch": (I32, [P, P, P, U64, U64, P]),
        "rlh_forward_into": (I32, [P, P, P, U64, U64, P]),
        "rlh_greedy_next": (I32, [P, P, ctypes.POINTER(U32)]),
        "rlh_generate_greedy": (I32, [P, P, U32, U64, P]),
        "rlh_sampler_init": (U64, [U64]),
        "rlh_softmax": (I32, [P, U64]),
        "rlh_sample": (I32, [P, U64, ctypes.POINTER(SamplingParams), P, U64, ctypes.POINTER(U64),
                             ctypes.POINTER(U32)]),
        "rlh_sample_next": (I32, [P, P, ctypes.POINTER(SamplingParams), P, U64, ctypes.POINTER(U64),
                                  ctypes.POINTER(U32)]),
        "rlh_generate": (I32, [P, P, P, U64, U64, ctypes.POINTER(SamplingParams), U32, P, ctypes.POINTER(U64)]),
        "rlh_cache_set_debug": (I32, [P, I32]),
        "rlh_debug_layer_hidden": (I32, [P, I32, P, U64]),
        "rlh_cache_read_kv": (I32, [P, I32, I32, U64, P]),
        "rlh_quantize_q8": (I32, [P, U64, P, P, P, P]),
        "rlh_dequant": (I32, [U32, P, U64, P]),
        "rlh_matvec": (I32, [U32, P, U64, U64, P, P]),
        "rlh_matmul_batch": (I32, [U32, P, U64, U64, P, U64, P]),
        "rlh_block_dots": (I32, [U32, P, U64, U64, P, P]),
        "rlh_argmax_noalloc": (I32, [P, U64, P, P]),
        "rlh_dsampler_create": (I32, [U64, ctypes.POINTER(P)]),
        "rlh_dsampler_destroy": (None, [P]),
        "rlh_dsampler_sample": (I32, [P, P, U64, ctypes.POINTER(SamplingParams), P, U64, ctypes.POINTER(U64),
                                      ctypes.POINTER(U32), P]),
        "rlh_dsampler_softmax": (I32, [P, P, U64, P]),
        "rlh_dsampler_set_candidate_cap": (I32, [P, U32]),
        "rlh_dsampler_last_path": (U32, [P]),
        "rlh_profile_matvec": (I32, [P, P, I32, I32, ctypes.POINTER(ctypes.c_double)]),
        "rlh_profile_decode": (I32, [P, P, I32, ctypes.POINTER(ctypes.c_double)]),
        "rlh_profile_decode_kernel": (I32, [P, P, I32, U32, I32, ctypes.POINTER(ctypes.c_double),
                                            ctypes.POINTER(U64)]),
        "rlh_gguf_open": (I32, [ctypes.c_char_p, ctypes.POINTER(P)]),
        "rlh_gguf_close": (None, [P]),
        "rlh_gguf_version": (U32, [P]),
        "rlh_gguf_n_files": (U64, [P]),
        "rlh_gguf_n_tensors": (U64, [P]),
        "rlh_gguf_tensor_info": (I32, [P, U64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(U32),
                                       ctypes.POINTER(U32), P, U32, ctypes.POINTER(U64), ctypes.POINTER(U32)]),
        "rlh_gguf_tensor_bytes": (I32, [P, ctypes.c_char_p, ctypes.POINTER(P), ctypes.POINTER(U64)]),
        "rlh_gguf_n_meta": (U64, [P]),
        "rlh_gguf_meta_key": (I32, [P, U64, ctypes.POINTER(ctypes.c_char_p)]),
        "rlh_gguf_meta_type": (I32, [P, ctypes.c_char_p, ctypes.POINTER(U32), ctypes.POINTER(U32),
                                     ctypes.POINTER(U64)]),
        "rlh_gguf_meta_u32": (I32, [P, ctypes.c_char_p, ctypes.POINTER(U32)]),
        "rlh_gguf_meta_f32": (I32, [P, ctypes.c_char_p, ctypes.POINTER(F)]),
        "rlh_gguf_meta_scalar": (I32, [P, ctypes.c_char_p, ctypes.POINTER(U64), ctypes.POINTER(ctypes.c_int64),
                                       ctypes.POINTER(ctypes.c_double)]),
        "rlh_gguf_meta_str": (I32, [P, ctypes.c_char_p, ctypes.POINTER(P), ctypes.POINTER(U64)]),
        "rlh_gguf_meta_arr_str": (I32, [P, ctypes.c_char_p, U64, ctypes.POINTER(P), ctypes.POINTER(U64)]),
        "rlh_gguf_meta_arr_scalar": (I32, [P, ctypes.c_char_p, U64, ctypes.POINTER(U64),
                                           ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_double)]),
        "rlh_gguf_config": (I32, [P, ctypes.POINTER(Config), ctypes.c_char_p, U64]),
        "rlh_model_load_gguf": (I32, [P, ctypes.POINTER(P)]),
        "rlh_gguf_writer_create": (I32, [U32, U64, ctypes.POINTER(P)]),
        "rlh_gguf_writer_destroy": (None, [P]),
        "rlh_gguf_writer_set_scalar": (I32, [P, ctypes.c_char_p, U32, P]),
        "rlh_gguf_writer_set_string": (I32, [P, ctypes.c_char_p, ctypes.c_char_p, U64]),
        "rlh_gguf_writer_set_array": (I32, [P, ctypes.c_char_p, U32, P, U64]),
        "rlh_gguf_writer_add_tensor": (I32, [P, ctypes.c_char_p, U32, U32, P, P, U64]),
        "rlh_gguf_writer_write": (I32, [P, ctypes.c_char_p]),
        "rlh_prune_vocab": (I32, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(PruneStats)]),
        "rlh_tokenizer_create": (I32, [P, U64, P, U64, P, U64, U32, U32, ctypes.POINTER(P)]),
        "rlh_tokenizer_from_gguf": (I32, [P, ctypes.POINTER(P)]),
        "rlh_tokenizer_destroy": (None, [P]),
        "rlh_tokenizer_vocab_size": (U64, [P]),
        "rlh_tokenizer_bos": (U32, [P]),
        "rlh_tokenizer_eos": (U32, [P]),
        "rlh_tokenizer_encode": (I32, [P, ctypes.c_char_p, U64, P, U64, ctypes.POINTER(U64)]),
        "rlh_tokenizer_pretokenize": (I32, [P, ctypes.c_char_p, U64, P, U64, ctypes.POINTER(U64)]),
        "rlh_tokenizer_decode": (I32, [P, P, U64, P, U64, ctypes.POINTER(U64)]),
        "rlh_tokenizer_token_bytes": (I32, [P, U32, P, U64, ctypes.POINTER(U64)]),
        "rlh_format_qwen_chat": (I32, [P, P, U64, ctypes.c_char_p, ctypes.c_char_p, I32, P, U64,
                                       ctypes.POINTER(U64)]),
        "rlh_quantize_row": (I32, [U32, P, U64, P]),
        "rlh_synth_normal": (None, [U64, U64, U64, U64, F, F, P]),
        "rlh_synth_tensor": (I32, [U64, U64, U32, U64, U64, F, F, P, I32]),
        "rlh_synth_tokens": (None, [U64, U64, U32, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class Sampler:
    """Sampler (src/sampler.rs:29-163) over host logits."""

    def __init__(self, seed):
        self.lib = load()
        self.state = ctypes.c_uint64(self.lib.rlh_sampler_init(seed))

    def sample(self, logits, params, recent):
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        r = np.ascontiguousarray(recent, dtype=np.uint32)
        t = ctypes.c_uint32()
        check(self.lib.rlh_sample(lg.ctypes.data, len(lg), ctypes.byref(params), r.ctypes.data, len(r),
                                  ctypes.byref(self.state), ctypes.byref(t)))
        return t.value


DSAMPLER_PATH_GREEDY, DSAMPLER_PATH_CANDIDATES, DSAMPLER_PATH_SORT, DSAMPLER_PATH_FALLBACK = 1, 2, 4, 8


class DeviceSampler:
    """Sampler (src/sampler.rs:29-163) over device-resident logits
    (rlh_dsampler_*): `logits` is a device address (e.g. a torch tensor's
    data_ptr()) of n float32 values; the RNG state lives on the host as in
    Sampler and advances identically."""

    def __init__(self, seed, max_n):
        self.lib = load()
        self.state = ctypes.c_uint64(self.lib.rlh_sampler_init(seed))
        h = ctypes.c_void_p()
        check(self.lib.rlh_dsampler_create(max_n, ctypes.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            self.lib.rlh_dsampler_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def sample(self, logits, n, params, recent, stream=None):
        r = np.ascontiguousarray(recent, dtype=np.uint32)
        t = ctypes.c_uint32()
        check(self.lib.rlh_dsampler_sample(self.h, logits, n, ctypes.byref(params), r.ctypes.data, len(r),
                                           ctypes.byref(self.state), ctypes.byref(t), stream))
        return t.value

    def softmax(self, x, n, stream=None):
        check(self.lib.rlh_dsampler_softmax(self.h, x, n, stream))

    def set_candidate_cap(self, cap):
        check(self.lib.rlh_dsampler_set_candidate_cap(self.h, cap))

    @property
    def last_path(self):
        return self.lib.rlh_dsampler_last_path(self.h)


class RlhError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"rlh error {code}: {msg}")
        self.code = code


def check(rc):
    if rc != 0:
        raise RlhError(rc, load().rlh_last_error().decode())
    return rc


def _p(a):
    return None if a is None else a.ctypes.data


class Model:
    """Device-resident model (Model, src/model.rs:136-239)."""

    def __init__(self, spec, tensors):
        self.lib = load()
        self.spec = spec
        cfg = spec.config()
        h = ctypes.c_void_p()
        check(self.lib.rlh_model_create(ctypes.byref(cfg), ctypes.byref(h)))
        self.h = h
        for kind, layer, ty, cols, rows, buf in tensors:
            check(self.lib.rlh_model_set_tensor(self.h, kind, layer, ty, buf.ctypes.data, cols, rows))
        check(self.lib.rlh_model_finalize(self.h))

    def close(self):
        if self.h:
            self.lib.rlh_model_destroy(self.h)
            self.h = None

    def new_cache(self, max_ctx):
        return Cache(self, max_ctx)


class Cache:
    """Device KV cache + stream (KvCache, src/model.rs:107-134)."""

    def __init__(self, model, max_ctx):
        self.lib = model.lib
        self.model = model
        h = ctypes.c_void_p()
        check(self.lib.rlh_cache_create(model.h, max_ctx, ctypes.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            self.lib.rlh_cache_destroy(self.h)
            self.h = None

    @property
    def len(self):
        return self.lib.rlh_cache_len(self.h)

    @property
    def max_ctx(self):
        return self.lib.rlh_cache_max_ctx(self.h)

    def reset(self):
        check(self.lib.rlh_cache_reset(self.h))

    def forward_into(self, tokens, start_pos, logits=None, copy=True):
        """Model::forward_into; returns the last token's logits (None when
        copy is False: the device keeps them for greedy_next / sample_next)."""
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        if copy and logits is None:
            logits = np.empty(self.model.spec.vocab, dtype=np.float32)
        check(self.lib.rlh_forward_into(self.model.h, self.h, toks.ctypes.data, len(toks), start_pos,
                                        logits.ctypes.data if copy else None))
        return logits if copy else None

    def greedy_next(self):
        t = ctypes.c_uint32()
        check(self.lib.rlh_greedy_next(self.model.h, self.h, ctypes.byref(t)))
        return t.value

    def sample_next(self, params, recent, state):
        """Sampler::sample on the logits of the last forward call
        (rlh_sample_next); `state` is a ctypes.c_uint64 RNG state."""
        r = np.ascontiguousarray(recent, dtype=np.uint32)
        t = ctypes.c_uint32()
        check(self.lib.rlh_sample_next(self.model.h, self.h, ctypes.byref(params), r.ctypes.data, len(r),
                                       ctypes.byref(state), ctypes.byref(t)))
        return t.value

    def generate_greedy(self, first, n_steps):
        out = np.empty(n_steps + 1, dtype=np.uint32)
        check(self.lib.rlh_generate_greedy(self.model.h, self.h, first, n_steps, out.ctypes.data))
        return out

    def generate(self, prompt, max_new, params, eos):
        """Model::generate (src/model.rs:741-776) on the device."""
        toks = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(max(1, max_new), dtype=np.uint32)
        n = ctypes.c_uint64()
        check(self.lib.rlh_generate(self.model.h, self.h, toks.ctypes.data, len(toks), max_new,
                                    ctypes.byref(params), eos, out.ctypes.data, ctypes.byref(n)))
        return out[: n.value].copy()

    def set_debug(self, on):
        check(self.lib.rlh_cache_set_debug(self.h, 1 if on else 0))

    def layer_hidden(self, layer, n_tokens):
        out = np.empty((n_tokens, self.model.spec.n_embd), dtype=np.float32)
        check(self.lib.rlh_debug_layer_hidden(self.h, layer, out.ctypes.data, n_tokens))
        return out

    def profile_matvec(self, kind, iters):
        v = ctypes.c_double()
        check(self.lib.rlh_profile_matvec(self.model.h, self.h, kind, iters, ctypes.byref(v)))
        return v.value

    def profile_decode_kernel(self, kind, first, steps):
        """(average microseconds per launch, launches timed) of one decode
        matvec kind inside `steps` greedy decode steps from token `first`."""
        v = ctypes.c_double()
        n = ctypes.c_uint64()
        check(self.lib.rlh_profile_decode_kernel(self.model.h, self.h, kind, first, steps, ctypes.byref(v),
                                                 ctypes.byref(n)))
        return v.value, n.value

    def profile_decode(self, iters):
        v = ctypes.c_double()
        check(self.lib.rlh_profile_decode(self.model.h, self.h, iters, ctypes.byref(v)))
        return v.value

    def read_kv(self, layer, which_v, n_pos):
        s = self.model.spec
        out = np.empty((n_pos, s.n_head_kv * s.head_dim), dtype=np.float32)
        check(self.lib.rlh_cache_read_kv(self.h, layer, which_v, n_pos, out.ctypes.data))
        return out


def quantize_q8(x):
    lib = load()
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = len(x)
    qs = np.empty(n, np.int8)
    d = np.empty(n // 32, np.float32)
    s = np.empty(n // 32, np.int32)
    s16 = np.empty(n // 16, np.int32)
    check(lib.rlh_quantize_q8(x.ctypes.data, n, qs.ctypes.data, d.ctypes.data, s.ctypes.data, s16.ctypes.data))
    return qs, d, s, s16


def dequant(ty, data, n):
    out = np.empty(n, np.float32)
    check(load().rlh_dequant(ty, np.ascontiguousarray(data).ctypes.data, n, out.ctypes.data))
    return out


def matvec(ty, w, rows, cols, x):
    y = np.empty(rows, np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    check(load().rlh_matvec(ty, np.ascontiguousarray(w).ctypes.data, rows, cols, x.ctypes.data, y.ctypes.data))
    return y


def block_dots(ty, w, rows, cols, q8):
    per = cols // 16 if ty == Q6_K else cols // 32
    out = np.empty((rows, per), np.int32)
    q8 = np.ascontiguousarray(q8, dtype=np.int8)
    check(load().rlh_block_dots(ty, np.ascontiguousarray(w).ctypes.data, rows, cols, q8.ctypes.data,
                                out.ctypes.data))
    return out


def matmul_batch(ty, w, rows, cols, xs, n):
    """ops::matmul_batch with integer semantics (BATCH_INT): ys[n][rows]."""
    ys = np.empty(n * rows, np.float32)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    check(load().rlh_matmul_batch(ty, np.ascontiguousarray(w).ctypes.data, rows, cols, xs.ctypes.data, n,
                                  ys.ctypes.data))
    return ys


# ---- GGUF files (src/gguf.rs, src/prune.rs:381-442) -------------------------

def gguf_tensor_name(kind, layer):
    """GGUF name of a tensor kind (Model::load's names, model.rs:164-218)."""
    base = KIND_NAMES[kind]
    suffix = ".bias" if kind in (T_ATTN_Q_BIAS, T_ATTN_K_BIAS, T_ATTN_V_BIAS) else ".weight"
    if base.endswith("_bias"):
        base = base[:-5]
    if kind in (T_TOKEN_EMBD, T_OUTPUT_NORM, T_OUTPUT):
        return base + suffix
    return f"blk.{layer}.{base}{suffix}"


class Gguf:
    """A GGUF file opened with rlh_gguf_open (GgufFile, gguf.rs:125-421)."""

    def __init__(self, path):
        self.lib = load()
        h = ctypes.c_void_p()
        check(self.lib.rlh_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            self.lib.rlh_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def version(self):
        return self.lib.rlh_gguf_version(self.h)

    @property
    def n_files(self):
        return self.lib.rlh_gguf_n_files(self.h)

    def tensors(self):
        """[(name, ggml type, dims, offset, file index)] in file order."""
        out = []
        for i in range(self.lib.rlh_gguf_n_tensors(self.h)):
            name, ty, nd = ctypes.c_char_p(), ctypes.c_uint32(), ctypes.c_uint32()
            dims = (ctypes.c_uint64 * 8)()
            off, fi = ctypes.c_uint64(), ctypes.c_uint32()
            check(self.lib.rlh_gguf_tensor_info(self.h, i, ctypes.byref(name), ctypes.byref(ty), ctypes.byref(nd),
                                                dims, 8, ctypes.byref(off), ctypes.byref(fi)))
            out.append((name.value.decode(), ty.value, [int(dims[k]) for k in range(min(nd.value, 8))],
                        off.value, fi.value))
        return out

    def tensor_bytes(self, name):
        """A copy of the tensor's bytes (uint8 array)."""
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        check(self.lib.rlh_gguf_tensor_bytes(self.h, name.encode(), ctypes.byref(p), ctypes.byref(n)))
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint8)), shape=(n.value,)).copy() \
            if n.value else np.zeros(0, np.uint8)

    def keys(self):
        out = []
        for i in range(self.lib.rlh_gguf_n_meta(self.h)):
            k = ctypes.c_char_p()
            check(self.lib.rlh_gguf_meta_key(self.h, i, ctypes.byref(k)))
            out.append(k.value.decode())
        return out

    def meta_type(self, key):
        t, e, n = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
        check(self.lib.rlh_gguf_meta_type(self.h, key.encode(), ctypes.byref(t), ctypes.byref(e), ctypes.byref(n)))
        return t.value, e.value, n.value

    def _scalar(self, ty, u, i, f):
        if ty in (GGUF_U8, GGUF_U16, GGUF_U32, GGUF_U64):
            return int(u)
        if ty in (GGUF_I8, GGUF_I16, GGUF_I32, GGUF_I64):
            return int(i)
        if ty == GGUF_BOOL:
            return bool(u)
        return float(f)

    def meta(self, key):
        """The value of a metadata key as a Python value (str, int, float,
        bool, or a list of them)."""
        ty, et, n = self.meta_type(key)
        kb = key.encode()
        if ty == GGUF_STR:
            p, ln = ctypes.c_void_p(), ctypes.c_uint64()
            check(self.lib.rlh_gguf_meta_str(self.h, kb, ctypes.byref(p), ctypes.byref(ln)))
            return ctypes.string_at(p, ln.value).decode("utf-8", "replace")
        u, i, f = ctypes.c_uint64(), ctypes.c_int64(), ctypes.c_double()
        if ty != GGUF_ARR:
            check(self.lib.rlh_gguf_meta_scalar(self.h, kb, ctypes.byref(u), ctypes.byref(i), ctypes.byref(f)))
            return self._scalar(ty, u.value, i.value, f.value)
        out = []
        for k in range(n):
            if et == GGUF_STR:
                p, ln = ctypes.c_void_p(), ctypes.c_uint64()
                check(self.lib.rlh_gguf_meta_arr_str(self.h, kb, k, ctypes.byref(p), ctypes.byref(ln)))
                out.append(ctypes.string_at(p, ln.value).decode("utf-8", "replace"))
            else:
                check(self.lib.rlh_gguf_meta_arr_scalar(self.h, kb, k, ctypes.byref(u), ctypes.byref(i),
                                                        ctypes.byref(f)))
                out.append(self._scalar(et, u.value, i.value, f.value))
        return out

    def config(self):
        """(Config, architecture) of Model::read_config (model.rs:241-293)."""
        c = Config()
        arch = ctypes.create_string_buffer(64)
        check(self.lib.rlh_gguf_config(self.h, ctypes.byref(c), arch, 64))
        return c, arch.value.decode()


def write_gguf(path, meta, tensors, version=3, alignment=32):
    """write_gguf (prune.rs:381-442). meta: {key: (gguf type, value)} where an
    array value is (GGUF_ARR, (element type, list)); tensors: [(name, ggml
    type, dims, bytes as a uint8 array)] with dims[0] the row length."""
    lib = load()
    w = ctypes.c_void_p()
    check(lib.rlh_gguf_writer_create(version, alignment, ctypes.byref(w)))
    keep = []
    try:
        for key, (ty, val) in meta.items():
            kb = key.encode()
            if ty == GGUF_STR:
                b = val.encode() if isinstance(val, str) else bytes(val)
                check(lib.rlh_gguf_writer_set_string(w, kb, b, len(b)))
            elif ty == GGUF_ARR:
                et, items = val
                if et == GGUF_STR:
                    bufs = [(x.encode() if isinstance(x, str) else bytes(x)) for x in items]
                    arr = (ctypes.c_char_p * max(1, len(bufs)))(*bufs)
                    keep.append((bufs, arr))
                    check(lib.rlh_gguf_writer_set_array(w, kb, et, arr, len(bufs)))
                else:
                    a = np.ascontiguousarray(np.array(items, dtype=_GGUF_NP[et]))
                    keep.append(a)
                    check(lib.rlh_gguf_writer_set_array(w, kb, et, a.ctypes.data if len(a) else None, len(a)))
            else:
                a = np.array([val], dtype=_GGUF_NP[ty])
                check(lib.rlh_gguf_writer_set_scalar(w, kb, ty, a.ctypes.data))
        for name, ty, dims, data in tensors:
            d = np.array(dims, np.uint64)
            buf = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
            keep.append((d, buf))
            check(lib.rlh_gguf_writer_add_tensor(w, name.encode(), ty, len(d), d.ctypes.data,
                                                 buf.ctypes.data if buf.size else None, buf.size))
        check(lib.rlh_gguf_writer_write(w, os.fsencode(path)))
    finally:
        lib.rlh_gguf_writer_destroy(w)


def prune_vocab(in_path, out_path):
    """prune::prune_vocab (prune.rs:127-291) through rlh_prune_vocab; returns
    the PruneStats counts as a dict."""
    lib = load()
    st = PruneStats()
    check(lib.rlh_prune_vocab(os.fsencode(in_path), os.fsencode(out_path), ctypes.byref(st)))
    return {f: getattr(st, f) for f, _ in PruneStats._fields_}


def model_gguf_meta(spec, n_ctx=None, vocab_tokens=None, extra=None):
    """Qwen3 metadata of a synthetic model (the keys Model::read_config and
    read_tokenizer read, model.rs:241-330). The vocabulary is placeholder
    strings unless given."""
    a = "qwen3"
    tokens = vocab_tokens if vocab_tokens is not None else [f"<t{i}>" for i in range(spec.vocab)]
    meta = {
        "general.architecture": (GGUF_STR, a),
        f"{a}.block_count": (GGUF_U32, spec.n_layer),
        f"{a}.embedding_length": (GGUF_U32, spec.n_embd),
        f"{a}.feed_forward_length": (GGUF_U32, spec.n_ff),
        f"{a}.attention.head_count": (GGUF_U32, spec.n_head),
        f"{a}.attention.head_count_kv": (GGUF_U32, spec.n_head_kv),
        f"{a}.attention.key_length": (GGUF_U32, spec.head_dim),
        f"{a}.attention.value_length": (GGUF_U32, spec.head_dim),
        f"{a}.rope.freq_base": (GGUF_F32, spec.rope_theta),
        f"{a}.attention.layer_norm_rms_epsilon": (GGUF_F32, spec.rms_eps),
        f"{a}.context_length": (GGUF_U32, n_ctx or spec.n_ctx),
        "tokenizer.ggml.model": (GGUF_STR, "gpt2"),
        "tokenizer.ggml.tokens": (GGUF_ARR, (GGUF_STR, tokens)),
        "tokenizer.ggml.token_type": (GGUF_ARR, (GGUF_I32, [1] * len(tokens))),
        "tokenizer.ggml.bos_token_id": (GGUF_U32, 0),
        "tokenizer.ggml.eos_token_id": (GGUF_U32, max(0, len(tokens) - 1)),
    }
    meta.update(extra or {})
    return meta


def model_gguf_tensors(tensors):
    """(name, type, dims, bytes) GGUF entries of synth_model's tensors."""
    return [(gguf_tensor_name(kind, layer), ty, [cols] if rows == 1 and kind not in (T_TOKEN_EMBD, T_OUTPUT)
             else [cols, rows], buf) for kind, layer, ty, cols, rows, buf in tensors]


def write_model_gguf(path, spec, tensors, **kw):
    """A synthetic model (synth_model's tensors) as one Qwen3 GGUF file."""
    write_gguf(path, model_gguf_meta(spec, **kw), model_gguf_tensors(tensors))


def load_model_gguf(path, spec=None):
    """Model::load through rlh_model_load_gguf; returns a Model whose spec is
    `spec` (or one built from the file's config)."""
    with Gguf(path) as g:
        lib = load()
        h = ctypes.c_void_p()
        check(lib.rlh_model_load_gguf(g.h, ctypes.byref(h)))
        if spec is None:
            c, _ = g.config()
            spec = ModelSpec("gguf", c.n_layer, c.n_embd, c.n_ff, c.n_head, c.n_head_kv, c.vocab_size,
                             not c.has_output, {}, c.head_dim, c.rope_theta, c.rms_eps, c.n_ctx)
    m = Model.__new__(Model)
    m.lib = lib
    m.spec = spec
    m.h = h
    return m


# ---- tokenizer and chat template (src/tokenizer.rs) -------------------------

def _cstr_array(items):
    bufs = [x.encode() if isinstance(x, str) else bytes(x) for x in items]
    return bufs, (ctypes.c_char_p * max(1, len(bufs)))(*bufs)


class Tokenizer:
    """The byte-level BPE tokenizer (Tokenizer, src/tokenizer.rs:34-359)."""

    def __init__(self, tokens=None, token_types=None, merges=None, bos=1, eos=2, gguf=None):
        self.lib = load()
        h = ctypes.c_void_p()
        if gguf is not None:
            check(self.lib.rlh_tokenizer_from_gguf(gguf.h, ctypes.byref(h)))
        else:
            tb, ta = _cstr_array(tokens)
            mb, ma = _cstr_array(merges or [])
            ty = np.ascontiguousarray(token_types if token_types is not None else [], np.uint32)
            check(self.lib.rlh_tokenizer_create(ta, len(tb), ty.ctypes.data if len(ty) else None, len(ty),
                                                ma, len(mb), bos, eos, ctypes.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            self.lib.rlh_tokenizer_destroy(self.h)
            self.h = None

    @property
    def vocab_size(self):
        return self.lib.rlh_tokenizer_vocab_size(self.h)

    @property
    def bos(self):
        return self.lib.rlh_tokenizer_bos(self.h)

    @property
    def eos(self):
        return self.lib.rlh_tokenizer_eos(self.h)

    def encode(self, text):
        b = text.encode() if isinstance(text, str) else bytes(text)
        n = ctypes.c_uint64()
        rc = self.lib.rlh_tokenizer_encode(self.h, b, len(b), None, 0, ctypes.byref(n))
        if rc != 0 and n.value == 0:
            check(rc)
        out = np.zeros(max(1, n.value), np.uint32)
        check(self.lib.rlh_tokenizer_encode(self.h, b, len(b), out.ctypes.data, len(out), ctypes.byref(n)))
        return [int(x) for x in out[:n.value]]

    def pretokenize(self, text):
        b = text.encode() if isinstance(text, str) else bytes(text)
        n = ctypes.c_uint64()
        rc = self.lib.rlh_tokenizer_pretokenize(self.h, b, len(b), None, 0, ctypes.byref(n))
        if rc != 0 and n.value == 0:
            check(rc)
        bounds = np.zeros(max(2, 2 * n.value), np.uint64)
        check(self.lib.rlh_tokenizer_pretokenize(self.h, b, len(b), bounds.ctypes.data, len(bounds),
                                                 ctypes.byref(n)))
        return [b[int(bounds[2 * k]):int(bounds[2 * k + 1])].decode() for k in range(n.value)]

    def _bytes_call(self, fn, *args):
        n = ctypes.c_uint64()
        fn(self.h, *args, None, 0, ctypes.byref(n))
        buf = ctypes.create_string_buffer(n.value + 1)
        check(fn(self.h, *args, buf, n.value + 1, ctypes.byref(n)))
        return buf.raw[:n.value]

    def decode(self, ids):
        a = np.ascontiguousarray(ids, np.uint32)
        return self._bytes_call(self.lib.rlh_tokenizer_decode, a.ctypes.data if len(a) else None,
                                len(a)).decode("utf-8")

    def token_bytes(self, token_id):
        return self._bytes_call(self.lib.rlh_tokenizer_token_bytes, token_id)


def format_qwen_chat(prompt, system=None, no_think=False, turns=()):
    """format_qwen_chat / format_qwen_multiturn (tokenizer.rs:386-430)."""
    lib = load()
    rb, ra = _cstr_array([r for r, _ in turns])
    cb, ca = _cstr_array([c for _, c in turns])
    n = ctypes.c_uint64()
    args = (ra, ca, len(turns), prompt.encode(), system.encode() if system is not None else None,
            1 if no_think else 0)
    lib.rlh_format_qwen_chat(*args, None, 0, ctypes.byref(n))
    buf = ctypes.create_string_buffer(n.value + 1)
    check(lib.rlh_format_qwen_chat(*args, buf, n.value + 1, ctypes.byref(n)))
    return buf.raw[:n.value].decode()
