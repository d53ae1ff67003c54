"""ctypes binding of the CPU oracle (liboracle.so, oracle/cpu_ref.h).

TEST INFRASTRUCTURE ONLY: the parity reference and the CPU baseline. Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

MODE_DEFAULT, MODE_NO_INT, MODE_BATCH_INT, MODE_NO_SIMD = 0, 1, 2, 4
MODE_SPLIT_ATTN = 8  # not a reference mode: split-K summation order in decode attention


class OrcConfig(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_uint32), ("n_embd", ctypes.c_uint32), ("n_ff", ctypes.c_uint32),
                ("n_head", ctypes.c_uint32), ("n_head_kv", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
                ("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float), ("n_ctx", ctypes.c_uint32),
                ("vocab_size", ctypes.c_uint32), ("has_qk_norm", ctypes.c_uint32), ("has_output", ctypes.c_uint32)]


class SamplingParams(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_uint32), ("top_p", ctypes.c_float),
                ("repetition_penalty", ctypes.c_float), ("repeat_last_n", ctypes.c_uint32),
                ("seed", ctypes.c_uint64)]


class BenchResult(ctypes.Structure):
    _fields_ = [("prefill_s", ctypes.c_double), ("decode_s", ctypes.c_double), ("prompt_len", ctypes.c_size_t),
                ("generated", ctypes.c_size_t)]


_lib = None


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: run `make -C oracle`")
    lib = ctypes.CDLL(LIB_PATH)
    P, U32, U64, SZ, I32, F = (ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_size_t, ctypes.c_int,
                               ctypes.c_float)
    sig = {
        "orc_type_block_size": (I32, [U32]), "orc_type_size": (I32, [U32]),
        "orc_f16_to_f32": (F, [ctypes.c_uint16]), "orc_f16_to_f32_scalar": (F, [ctypes.c_uint16]),
        "orc_get_scale_min_k4": (None, [I32, P, P, P]),
        "orc_dequant_row": (I32, [U32, P, SZ, P]),
        "orc_dequant_dot_scalar": (F, [U32, P, P, SZ]), "orc_dequant_dot": (F, [U32, P, P, SZ]),
        "orc_simd_available": (I32, []),
        "orc_quantize_q8": (None, [P, SZ, I32, P, P, P, P]),
        "orc_dot_qk_q8_row": (I32, [U32, P, SZ, P, P, P, P, P]),
        "orc_block_dots": (I32, [U32, P, SZ, P, P]),
        "orc_rmsnorm_avx2": (None, [P, P, P, SZ, F]),
        "orc_dot_f32_avx2": (F, [P, P, SZ]),
        "orc_saxpy_avx2": (None, [P, F, P, SZ]),
        "orc_dot_multi": (None, [P, SZ, P, SZ, SZ, SZ, P, SZ]),
        "orc_dot_multi_rows_3_4": (None, [P, SZ, P, SZ, SZ, P, SZ]),
        "orc_split_dequant": (I32, [U32, P, SZ, P]),
        "orc_set_threads": (None, [I32]), "orc_get_threads": (I32, []),
        "orc_dot": (F, [P, P, SZ]),
        "orc_matmul": (None, [U32, P, SZ, SZ, P, P, I32]),
        "orc_matmul_batch": (None, [U32, P, SZ, SZ, P, SZ, P, I32]),
        "orc_rmsnorm": (None, [P, P, P, SZ, F, I32]),
        "orc_rmsnorm_head": (None, [P, P, SZ, F, I32]),
        "orc_silu": (F, [F]), "orc_softmax_inplace": (None, [P, SZ]),
        "orc_rope_neox_freqs": (None, [P, SZ, SZ, SZ, P]),
        "orc_model_create": (P, [ctypes.POINTER(OrcConfig)]),
        "orc_model_set_tensor": (I32, [P, I32, I32, U32, P, SZ, SZ]),
        "orc_model_finalize": (I32, [P]), "orc_model_destroy": (None, [P]),
        "orc_cache_create": (P, [P, SZ]), "orc_cache_reset": (None, [P]),
        "orc_cache_len": (SZ, [P]), "orc_cache_max_ctx": (SZ, [P]), "orc_cache_destroy": (None, [P]),
        "orc_forward_into": (None, [P, P, P, SZ, SZ, P, I32]),
        "orc_set_hidden_dump": (None, [P, P, SZ]),
        "orc_cache_k": (P, [P, I32]), "orc_cache_v": (P, [P, I32]),
        "orc_sampler_create": (P, [U64]), "orc_sampler_destroy": (None, [P]),
        "orc_sampler_next_u64": (U64, [P]), "orc_sampler_next_f32": (F, [P]),
        "orc_sampler_sample": (U32, [P, P, SZ, ctypes.POINTER(SamplingParams), P, SZ]),
        "orc_argmax": (U32, [P, SZ]),
        "orc_generate": (SZ, [P, P, P, SZ, SZ, ctypes.POINTER(SamplingParams), U32, P, I32]),
        "orc_bench": (I32, [P, P, P, SZ, SZ, I32, I32, ctypes.POINTER(BenchResult), P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    lib.orc_set_threads(default_threads())
    _lib = lib
    return lib


def default_threads():
    """Worker threads of the oracle's pool: the CPUs this process may run
    on (what rayon's default pool takes, std::thread::available_parallelism),
    capped at 16, the host share that goes with one GPU."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def quantize_q8(x, mode=0):
    """simd::quantize_q8 (mode 0 dispatch, 1 AVX2, 2 scalar)."""
    lib = load()
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = len(x)
    qs = np.empty(n, np.int8)
    d = np.empty(n // 32, np.float32)
    s = np.empty(n // 32, np.int32)
    s16 = np.empty(n // 16, np.int32)
    lib.orc_quantize_q8(x.ctypes.data, n, mode, qs.ctypes.data, d.ctypes.data, s.ctypes.data, s16.ctypes.data)
    return qs, d, s, s16


def dequant_row(ty, data, n):
    out = np.empty(n, np.float32)
    rc = load().orc_dequant_row(ty, np.ascontiguousarray(data).ctypes.data, n, out.ctypes.data)
    assert rc == 0
    return out


def dot_qk_q8_row(ty, row, q8):
    qs, d, s, s16 = q8
    out = ctypes.c_float()
    rc = load().orc_dot_qk_q8_row(ty, np.ascontiguousarray(row).ctypes.data, len(qs), qs.ctypes.data,
                                  d.ctypes.data, s.ctypes.data, s16.ctypes.data, ctypes.byref(out))
    assert rc == 0
    return np.float32(out.value)


def block_dots(ty, w, rows, cols, q8):
    from_row = w.reshape(rows, -1)
    per = cols // 16 if ty == 14 else cols // 32
    out = np.empty((rows, per), np.int32)
    lib = load()
    q8 = np.ascontiguousarray(q8, dtype=np.int8)
    for r in range(rows):
        row = np.ascontiguousarray(from_row[r])
        o = np.empty(per, np.int32)
        assert lib.orc_block_dots(ty, row.ctypes.data, cols, q8.ctypes.data, o.ctypes.data) == 0
        out[r] = o
    return out


def matmul(ty, w, rows, cols, x, mode=MODE_DEFAULT):
    y = np.empty(rows, np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    load().orc_matmul(ty, np.ascontiguousarray(w).ctypes.data, rows, cols, x.ctypes.data, y.ctypes.data, mode)
    return y


def matmul_batch(ty, w, rows, cols, xs, n, mode=MODE_DEFAULT):
    ys = np.empty(n * rows, np.float32)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    load().orc_matmul_batch(ty, np.ascontiguousarray(w).ctypes.data, rows, cols, xs.ctypes.data, n,
                            ys.ctypes.data, mode)
    return ys


class OracleModel:
    """CPU reference model over the same tensor bytes (keeps them alive)."""

    def __init__(self, spec, tensors):
        self.lib = load()
        self.spec = spec
        cfg = OrcConfig(spec.n_layer, spec.n_embd, spec.n_ff, spec.n_head, spec.n_head_kv, spec.head_dim,
                        spec.rope_theta, spec.rms_eps, spec.n_ctx, spec.vocab, 1, 0 if spec.tied else 1)
        self.h = self.lib.orc_model_create(ctypes.byref(cfg))
        self._keep = []
        for kind, layer, ty, cols, rows, buf in tensors:
            self._keep.append(buf)
            rc = self.lib.orc_model_set_tensor(self.h, kind, layer, ty, buf.ctypes.data, cols, rows)
            assert rc == 0, (kind, layer, rc)
        assert self.lib.orc_model_finalize(self.h) == 0

    def close(self):
        if self.h:
            self.lib.orc_model_destroy(self.h)
            self.h = None

    def new_cache(self, max_ctx):
        return OracleCache(self, max_ctx)


class OracleCache:
    def __init__(self, model, max_ctx):
        self.model = model
        self.lib = model.lib
        self.h = self.lib.orc_cache_create(model.h, max_ctx)
        self._dump = None

    def close(self):
        if self.h:
            self.lib.orc_cache_destroy(self.h)
            self.h = None

    @property
    def len(self):
        return self.lib.orc_cache_len(self.h)

    def reset(self):
        self.lib.orc_cache_reset(self.h)

    def enable_dump(self, max_tokens):
        s = self.model.spec
        self._dump = np.zeros((s.n_layer, max_tokens, s.n_embd), np.float32)
        self.lib.orc_set_hidden_dump(self.h, self._dump.ctypes.data, max_tokens)

    def hidden(self, layer, n_tokens):
        return self._dump[layer, :n_tokens].copy()

    def forward_into(self, tokens, start_pos, mode=MODE_BATCH_INT):
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.empty(self.model.spec.vocab, np.float32)
        self.lib.orc_forward_into(self.model.h, self.h, toks.ctypes.data, len(toks), start_pos,
                                  logits.ctypes.data, mode)
        return logits

    def read_kv(self, layer, which_v, n_pos):
        s = self.model.spec
        kvd = s.n_head_kv * s.head_dim
        p = self.lib.orc_cache_v(self.h, layer) if which_v else self.lib.orc_cache_k(self.h, layer)
        arr = np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), shape=(n_pos * kvd,))
        return arr.reshape(n_pos, kvd).copy()

    def generate(self, prompt, max_new, params, eos, mode=MODE_BATCH_INT):
        """Model::generate (model.rs:741-776); returns the generated tokens."""
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(max(1, max_new), np.uint32)
        n = self.lib.orc_generate(self.model.h, self.h, p.ctypes.data, len(p), max_new, ctypes.byref(params), eos,
                                  out.ctypes.data, mode)
        return out[:n].copy()

    def bench(self, prompt, n_gen, mode=MODE_DEFAULT, warmup=True):
        """main.rs cmd_bench protocol; returns (BenchResult, tokens)."""
        res = BenchResult()
        toks = np.empty(n_gen + 1, np.uint32)
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        rc = self.lib.orc_bench(self.model.h, self.h, p.ctypes.data, len(p), n_gen, mode, 1 if warmup else 0,
                                ctypes.byref(res), toks.ctypes.data)
        assert rc == 0
        return res, toks[:res.generated + 1]
