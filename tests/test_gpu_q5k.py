"""Q5_K on the device: the reference has no integer kernel for it, so
ops::matmul uses the fused f32 dequant-dot (quant.rs:528-539: per 256-value
block, dot_f32_avx2 of the dequantized block against the f32 activation,
summed in order) and ops::matmul_batch the f32 route (dequant rows +
dot_multi_rows, ops.rs:237-312). Bar: bit-exact against the oracle, which
restates those paths."""
import numpy as np
import pytest

import oracle
import rlh
from helpers import Q5_K, bits, random_blocks

pytestmark = pytest.mark.gpu


def test_dequant_q5k_bit_exact():
    rng = np.random.default_rng(13)
    n = 4096
    data = random_blocks(Q5_K, n // 256, rng)
    assert np.array_equal(bits(rlh.dequant(Q5_K, data, n)), bits(oracle.dequant_row(Q5_K, data, n)))


@pytest.mark.parametrize("rows,cols", [(1, 256), (5, 512), (33, 2048), (100, 2560), (20, 4096), (7, 12288),
                                       (9, 25600)])
def test_matvec_q5k_bit_exact(rows, cols):
    print(f"q5k matvec {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows * 3 + cols)
    w = random_blocks(Q5_K, rows * cols // 256, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    got = rlh.matvec(Q5_K, w, rows, cols, x)
    ref = oracle.matmul(Q5_K, w, rows, cols, x, oracle.MODE_DEFAULT)
    assert np.array_equal(bits(got), bits(ref)), f"max diff {np.max(np.abs(got - ref))}"


@pytest.mark.parametrize("rows,cols,n", [(16, 256, 2), (33, 1024, 5), (20, 2048, 16), (40, 4096, 35),
                                         (17, 12288, 7), (64, 512, 130)])
def test_matmul_batch_q5k_bit_exact(rows, cols, n):
    """Token groups of 4 (8-lane chains) and the n % 4 tail (dot_f32_avx2)."""
    print(f"q5k matmul_batch {rows}x{cols} n={n}", flush=True)
    rng = np.random.default_rng(rows + cols * 5 + n)
    w = random_blocks(Q5_K, rows * cols // 256, rng)
    xs = rng.standard_normal(n * cols).astype(np.float32)
    got = rlh.matmul_batch(Q5_K, w, rows, cols, xs, n)
    ref = oracle.matmul_batch(Q5_K, w, rows, cols, xs, n, oracle.MODE_BATCH_INT)
    assert np.array_equal(bits(got), bits(ref))


def test_forward_q5km_bit_exact():
    """A model with Q5_K matrices (and a tied Q5_K embedding / logits
    matrix): prefill of 13 tokens (3 in the n % 4 tail), then decode."""
    spec = rlh.SPECS["tiny-q5km"]
    tensors = rlh.synth_model(spec, 5151)
    m = rlh.Model(spec, tensors)
    om = oracle.OracleModel(spec, tensors)
    prompt = rlh.synth_tokens(52, 13, spec.vocab)
    c = m.new_cache(64)
    oc = om.new_cache(64)
    lg = c.forward_into(prompt, 0)
    rg = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    assert np.array_equal(bits(lg), bits(rg))
    lib = oracle.load()
    tok = lib.orc_argmax(rg.ctypes.data, len(rg))
    for i in range(6):
        lg = c.forward_into(np.array([tok], np.uint32), len(prompt) + i)
        rg = oc.forward_into(np.array([tok], np.uint32), len(prompt) + i, oracle.MODE_DEFAULT)
        assert np.array_equal(bits(lg), bits(rg)), f"decode step {i}"
        tok = lib.orc_argmax(rg.ctypes.data, len(rg))
    for l in range(spec.n_layer):
        for which in (0, 1):
            n = len(prompt) + 6
            assert np.array_equal(bits(c.read_kv(l, which, n)), bits(oc.read_kv(l, which, n)))
    c.close()
    oc.close()
    m.close()
