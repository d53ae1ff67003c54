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


def test_pruned_model_decodes_like_the_oracle(tmp_path):
    """prune_vocab (prune.rs:127-291) on a synthetic model whose vocabulary
    is one third CJK: the pruned file loads onto the device and decodes
    bit-exact against the oracle over the pruned tensors (token_embd and
    output hold only the kept rows), and its logits are the unpruned model's
    logits at the kept ids, for the same prompt."""
    import prune_ref

    spec = rlh.SPECS["tiny-q4km-untied"]
    tensors = rlh.synth_model(spec, 80)
    # byte-level token strings: "w<i>", or a CJK character for every third id
    b2u = {b: ch for ch, b in prune_ref._U2B.items()}
    vocab = ["".join(b2u[b] for b in (f"w{i}" if i % 3 else chr(0x4E00 + i)).encode()) for i in range(spec.vocab)]
    src, dst = tmp_path / "full.gguf", tmp_path / "pruned.gguf"
    rlh.write_model_gguf(src, spec, tensors, vocab_tokens=vocab)
    st = rlh.prune_vocab(src, dst)
    keep = [i for i in range(spec.vocab) if i % 3 or i == 0]  # id 0 is the bos token: pinned
    assert st["new_vocab"] == len(keep) and st["dropped"] == spec.vocab - len(keep)
    new_spec = rlh.ModelSpec("pruned", spec.n_layer, spec.n_embd, spec.n_ff, spec.n_head, spec.n_head_kv,
                             len(keep), spec.tied, spec.types, spec.head_dim, spec.rope_theta, spec.rms_eps,
                             spec.n_ctx)
    pruned = []
    for kind, layer, ty, cols, rows, buf in tensors:
        if kind in (rlh.T_TOKEN_EMBD, rlh.T_OUTPUT):
            rb = len(buf) // rows
            buf = np.ascontiguousarray(buf.reshape(rows, rb)[keep]).reshape(-1)
            rows = len(keep)
        pruned.append((kind, layer, ty, cols, rows, buf))
    with rlh.Gguf(dst) as g:
        for kind, layer, ty, cols, rows, buf in pruned:
            assert np.array_equal(g.tensor_bytes(rlh.gguf_tensor_name(kind, layer)), buf)
    m = rlh.load_model_gguf(dst, new_spec)
    full = rlh.Model(spec, tensors)
    try:
        _decode_matches_oracle(m, new_spec, pruned)
        prompt_new = rlh.synth_tokens(42, 9, len(keep))
        prompt_old = np.array([keep[i] for i in prompt_new], np.uint32)
        c, cf = m.new_cache(16), full.new_cache(16)
        lp = c.forward_into(prompt_new, 0)
        lf = cf.forward_into(prompt_old, 0)
        assert np.array_equal(bits(lp), bits(lf[keep]))
        c.close()
        cf.close()
    finally:
        m.close()
        full.close()
