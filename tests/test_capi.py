"""The C-ABI library: loads, exports every entry point include/rlh.h declares,
and refuses loudly (an error code, no CPU fallback) when no GPU is present.
Runs without a GPU."""
import ctypes
import os
import re

import numpy as np
import pytest

import rlh

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "rlh.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rlh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for must in ["rlh_forward_one", "rlh_forward_batch", "rlh_forward_into", "rlh_cache_create",
                 "rlh_cache_reset", "rlh_model_set_tensor", "rlh_greedy_next", "rlh_quantize_q8",
                 "rlh_matvec", "rlh_matmul_batch", "rlh_block_dots", "rlh_dequant", "rlh_debug_layer_hidden"]:
        assert must in syms


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(rlh.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_row_bytes_matches_ggml_sizes():
    lib = rlh.load()
    assert lib.rlh_row_bytes(rlh.Q4_K, 4096) == 16 * 144
    assert lib.rlh_row_bytes(rlh.Q6_K, 12288) == 48 * 210
    assert lib.rlh_row_bytes(rlh.Q8_0, 1024) == 32 * 34
    assert lib.rlh_row_bytes(rlh.Q4_K, 100) == 0
    assert lib.rlh_row_bytes(99, 256) == 0


def _has_gpu():
    try:
        import torch

        return torch.cuda.device_count() > 0
    except Exception:
        return False


@pytest.mark.skipif(_has_gpu(), reason="checks the no-GPU error path")
def test_model_create_fails_loudly_without_gpu():
    lib = rlh.load()
    cfg = rlh.SPECS["tiny-q4km"].config()
    h = ctypes.c_void_p()
    rc = lib.rlh_model_create(ctypes.byref(cfg), ctypes.byref(h))
    assert rc == rlh.RLH_EDEVICE
    assert b"no HIP device" in lib.rlh_last_error()
    x = np.zeros(64, np.float32)
    with pytest.raises(rlh.RlhError):
        rlh.quantize_q8(x)


def test_invalid_arguments_return_codes():
    lib = rlh.load()
    assert lib.rlh_model_create(None, None) == rlh.RLH_EINVAL
    assert lib.rlh_forward_one(None, None, 0, 0, None) == rlh.RLH_EINVAL
    assert lib.rlh_cache_reset(None) == rlh.RLH_EINVAL
    assert lib.rlh_last_error() != b""
