"""Model::load from GGUF files on the device (rlh_gguf_open +
rlh_model_load_gguf, src/model.rs:150-293, src/gguf.rs:246-307): a seeded
synthetic model written as a Qwen3 GGUF — one file, and split in two files
— loads onto the device and decodes with logits bit-identical to the oracle
over the same tensor bytes."""
import numpy as np
import pytest

import oracle
import rlh
from helpers import bits

pytestmark = pytest.mark.gpu


def _decode_matches_oracle(m, spec, tensors, n_prompt=11, n_gen=6):
    om = oracle.OracleModel(spec, tensors)
    lib = oracle.load()
    prompt = rlh.synth_tokens(41, n_prompt, spec.vocab)
    c = m.new_cache(n_prompt + n_gen + 1)
    oc = om.new_cache(n_prompt + n_gen + 1)
    try:
        lg = c.forward_into(prompt, 0)
        rg = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
        assert np.array_equal(bits(lg), bits(rg)), "prefill logits differ"
        tok = lib.orc_argmax(rg.ctypes.data, len(rg))
        for i in range(n_gen):
            lg = c.forward_into(np.array([tok], np.uint32), n_prompt + i)
            rg = oc.forward_into(np.array([tok], np.uint32), n_prompt + i, oracle.MODE_DEFAULT)
            assert np.array_equal(bits(lg), bits(rg)), f"decode step {i} logits differ"
            tok = lib.orc_argmax(rg.ctypes.data, len(rg))
    finally:
        c.close()
        oc.close()
        om.close()


@pytest.mark.parametrize("name", ["tiny-q4km-untied", "tiny-q8_0", "qwen3-0.6b-q4km"])
def test_model_from_gguf_file(name, tmp_path):
    print(f"gguf load {name}", flush=True)
    spec = rlh.SPECS[name]
    tensors = rlh.synth_model(spec, 77)
    p = tmp_path / f"{name}.gguf"
    rlh.write_model_gguf(p, spec, tensors)
    m = rlh.load_model_gguf(p, spec)
    try:
        assert rlh.load().rlh_model_weight_bytes(m.h) > 0
        _decode_matches_oracle(m, spec, tensors)
    finally:
        m.close()


def test_model_from_split_gguf(tmp_path):
    """Two files, -00001-of-00002.gguf holding the metadata and the global
    tensors, -00002-of-00002.gguf the layers (gguf.rs:259-293)."""
    spec = rlh.SPECS["tiny-q4km"]
    tensors = rlh.synth_model(spec, 78)
    entries = rlh.model_gguf_tensors(tensors)
    first = [e for e in entries if not e[0].startswith("blk.")]
    rest = [e for e in entries if e[0].startswith("blk.")]
    meta = rlh.model_gguf_meta(spec, extra={"split.count": (rlh.GGUF_U16, 2)})
    base = tmp_path / "tiny"
    rlh.write_gguf(f"{base}-00001-of-00002.gguf", meta, first)
    rlh.write_gguf(f"{base}-00002-of-00002.gguf", {"split.count": (rlh.GGUF_U16, 2)}, rest)
    with rlh.Gguf(f"{base}-00001-of-00002.gguf") as g:
        assert g.n_files == 2
    m = rlh.load_model_gguf(f"{base}-00001-of-00002.gguf", spec)
    try:
        _decode_matches_oracle(m, spec, tensors)
    finally:
        m.close()


def test_missing_tensor_is_reported(tmp_path):
    """A file without one layer matrix fails to load with its name (the
    "missing required tensor" error of model.rs:41-52), leaving nothing
    behind."""
    spec = rlh.SPECS["tiny-q4km"]
    tensors = rlh.synth_model(spec, 79)
    entries = [e for e in rlh.model_gguf_tensors(tensors) if e[0] != "blk.1.ffn_up.weight"]
    p = tmp_path / "missing.gguf"
    rlh.write_gguf(p, rlh.model_gguf_meta(spec), entries)
    with pytest.raises(rlh.RlhError) as e:
        rlh.load_model_gguf(p, spec)
    assert e.value.code == rlh.RLH_ESTATE
    assert b"blk.1.ffn_up.weight" in rlh.load().rlh_last_error()
