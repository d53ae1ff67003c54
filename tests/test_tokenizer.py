"""librlh's byte-level BPE tokenizer and chat template (src/tokenizer.rs,
Model::read_tokenizer model.rs:295-330) against the reference's own tests and
two independent implementations: the Qwen2 pre-tokenizer regex run by the
`regex` module, and Hugging Face `tokenizers` BPE over a vocabulary it
trains. CPU only.

The reference writes the pre-tokenizer pattern out by hand; it differs from
the regex in one case, a whitespace run holding a line break, then other
whitespace, then another line break (the regex's `\\s*[\\r\\n]+` backtracks
over the inner line break, the reference's loop stops at it). The product
follows the reference there (test_whitespace_run_with_two_line_breaks)."""
import json
import random

import pytest
import regex

import rlh

QWEN2_PATTERN = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*"
                 r"|\s*[\r\n]+|\s+(?!\S)|\s+")
DEVIATION = regex.compile(r"[\r\n][^\S\r\n]+[\r\n]")
ALPHABET = list("abcdefXYZéñß中文字") + list("0123456789٣") + list(" .,;:!?'\"()[]-_/@#$%&*+=<>|") + \
    ["\n", "\t", " ", " ", "  ", "\n\n", "\r\n", "'s", "'ll", "'RE", "'t", "'M", "'d", "'ve"]


@pytest.fixture(scope="module")
def bare():
    t = rlh.Tokenizer(["x"], [], [], 0, 0)
    yield t
    t.close()


def _texts(seed, n, maxlen=24):
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        s = "".join(rng.choice(ALPHABET) for _ in range(rng.randint(1, maxlen)))
        if not DEVIATION.search(s):
            out.append(s)
    return out


def test_reference_pretokenize_cases(bare):
    """tokenizer.rs:439-456."""
    assert bare.pretokenize("a ,b") == ["a", " ,", "b"]
    assert bare.pretokenize("x (y)") == ["x", " (", "y", ")"]
    assert bare.pretokenize("hello world") == ["hello", " world"]
    assert bare.pretokenize("a\n\n b") == ["a", "\n\n", " b"]


def test_pretokenize_matches_the_qwen2_regex(bare):
    rx = regex.compile(QWEN2_PATTERN)
    for s in _texts(7, 4000):
        assert bare.pretokenize(s) == rx.findall(s), repr(s)


def test_whitespace_run_with_two_line_breaks(bare):
    """The reference's alt5 loop (tokenizer.rs:203-212) takes the run up to
    the first line break group."""
    assert bare.pretokenize("a\n \nb") == ["a", "\n", " \n", "b"]
    assert bare.pretokenize("x\t\t\n\n \ny") == ["x", "\t\t\n\n", " \n", "y"]


def test_character_classes(bare):
    """Rust's is_alphabetic / is_numeric / is_whitespace (tokenizer.rs:45-53):
    a combining vowel sign (Alphabetic, general category Mc) joins a letter
    run, a Roman numeral (Nl) and a superscript digit (No) are numbers, NBSP
    and U+3000 are spaces."""
    assert bare.pretokenize("कि") == ["कि"]       # U+0915 U+093F
    assert bare.pretokenize("1²") == ["1", "²"]
    assert bare.pretokenize("a b") == ["a", " b"]
    assert bare.pretokenize("a　　b") == ["a", "　", "　b"]


@pytest.fixture(scope="module")
def hf_pair():
    tokenizers = pytest.importorskip("tokenizers")
    from tokenizers import Regex, Tokenizer, models, pre_tokenizers, trainers

    hf = Tokenizer(models.BPE())
    hf.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(QWEN2_PATTERN), behavior="isolated"),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    trainer = trainers.BpeTrainer(vocab_size=900, initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                                  show_progress=False)
    rng = random.Random(3)
    words = ["the", "model", "token", "Qwen", "décodé", "中文字", "run", "fast", "GPU", "ROCm", "'s", "42", "don't"]
    corpus = [" ".join(rng.choice(words) for _ in range(12)) + rng.choice([".", "!", "?\n", ",", ""]) for _ in range(3000)]
    hf.train_from_iterator(corpus, trainer)
    model = json.loads(hf.to_str())["model"]
    vocab = model["vocab"]
    merges = [m if isinstance(m, str) else " ".join(m) for m in model["merges"]]
    tokens = [None] * len(vocab)
    for tok, i in vocab.items():
        tokens[i] = tok
    specials = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]
    types = [1] * len(tokens) + [3] * len(specials)
    ours = rlh.Tokenizer(tokens + specials, types, merges, 0, len(tokens) + 2)
    yield hf, ours, tokens, specials
    ours.close()


def test_encode_matches_hf_bpe(hf_pair):
    """Full encode (pre-tokenizer + byte-level BPE merges by rank) equals Hugging
    Face `tokenizers` over the same vocabulary and merges."""
    hf, ours, _, _ = hf_pair
    texts = _texts(11, 1500, 40) + ["the model runs fast on the GPU. Qwen's 中文字 don't décodé 42!"]
    for s in texts:
        assert ours.encode(s) == hf.encode(s).ids, repr(s)


def test_special_tokens_and_round_trip(hf_pair):
    """Special tokens (types 3/4) match verbatim, the longest first at one
    position (tokenizer.rs:299-327); decode(encode(text)) == text."""
    _, ours, tokens, specials = hf_pair
    base = len(tokens)
    text = rlh.format_qwen_chat("the model 中文字", system="fast GPU")
    ids = ours.encode(text)
    assert ids[0] == base + 1 and ids.count(base + 2) == 2 and ids.count(base + 1) == 3
    assert ours.decode(ids) == text
    for s in _texts(13, 300, 60):
        assert ours.decode(ours.encode(s)) == s
    assert ours.encode("x<|im_end|><|im_end|>y")[1:3] == [base + 2, base + 2]


def test_decode_is_lossy_utf8(hf_pair):
    """Decoding bytes that are not valid UTF-8 replaces each maximal invalid
    subpart with U+FFFD (String::from_utf8_lossy), as Python's "replace"."""
    _, ours, tokens, _ = hf_pair
    byte_id = {}
    for i in range(len(tokens)):
        b = ours.token_bytes(i)
        if len(b) == 1:
            byte_id.setdefault(b[0], i)
    assert len(byte_id) == 256
    rng = random.Random(5)
    for _ in range(500):
        raw = bytes(rng.choice([0x41, 0x80, 0xBF, 0xC2, 0xE0, 0xED, 0xF0, 0xF4, 0xF8, 0xA0, 0x9F, 0x90, 0x8F])
                    for _ in range(rng.randint(1, 12)))
        assert ours.decode([byte_id[b] for b in raw]) == raw.decode("utf-8", "replace"), raw
    assert ours.decode([10 ** 9]) == ""  # unknown ids are skipped


def test_bpe_merge_rules():
    """bpe (tokenizer.rs:270-297): the lowest rank merges first, the leftmost
    pair among equal ranks; a merge whose parts or result are not in the
    vocabulary is dropped; a repeated pair keeps its last rank."""
    toks = ["a", "b", "c", "ab", "bc", "abc"]
    t = rlh.Tokenizer(toks, [], ["b c", "a b", "ab c"], 0, 0)
    assert t.encode("abc") == [toks.index("a"), toks.index("bc")]  # "b c" has rank 0
    t2 = rlh.Tokenizer(toks, [], ["a b", "b c", "ab c"], 0, 0)
    assert t2.encode("abc") == [toks.index("abc")]
    t3 = rlh.Tokenizer(toks, [], ["a b", "x y", "b c", "a b"], 0, 0)  # "a b" re-ranked to 3, after "b c"
    assert t3.encode("abc") == [toks.index("a"), toks.index("bc")]
    t4 = rlh.Tokenizer(toks, [], ["a a"], 0, 0)
    assert t4.encode("aa") == [0, 0]  # "aa" is not in the vocabulary


def test_chat_templates():
    """format_qwen_chat / format_qwen_multiturn (tokenizer.rs:386-430)."""
    assert rlh.format_qwen_chat("hi") == "<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n"
    assert rlh.format_qwen_chat("hi", system="S", no_think=True) == (
        "<|im_start|>system\nS<|im_end|>\n<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n"
        "<think>\n\n</think>\n\n")
    assert rlh.format_qwen_chat("q2", turns=[("user", "q1"), ("assistant", "a1")]) == (
        "<|im_start|>user\nq1<|im_end|>\n<|im_start|>assistant\na1<|im_end|>\n"
        "<|im_start|>user\nq2<|im_end|>\n<|im_start|>assistant\n")


def test_tokenizer_from_gguf(tmp_path, hf_pair):
    """Model::read_tokenizer (model.rs:295-330): tokens, token types, merges,
    bos/eos ids from GGUF metadata (types default to 1, ids to 1 and 2)."""
    hf, ours, tokens, specials = hf_pair
    model = json.loads(hf.to_str())["model"]
    merges = [m if isinstance(m, str) else " ".join(m) for m in model["merges"]]
    meta = {"tokenizer.ggml.tokens": (rlh.GGUF_ARR, (rlh.GGUF_STR, tokens + specials)),
            "tokenizer.ggml.token_type": (rlh.GGUF_ARR, (rlh.GGUF_I32, [1] * len(tokens) + [3] * len(specials))),
            "tokenizer.ggml.merges": (rlh.GGUF_ARR, (rlh.GGUF_STR, merges)),
            "tokenizer.ggml.eos_token_id": (rlh.GGUF_U32, len(tokens) + 2)}
    p = tmp_path / "tok.gguf"
    rlh.write_gguf(p, meta, [])
    with rlh.Gguf(p) as g:
        t = rlh.Tokenizer(gguf=g)
    assert t.vocab_size == len(tokens) + 3 and t.bos == 1 and t.eos == len(tokens) + 2
    s = "<|im_start|>user\nthe model's GPU<|im_end|>"
    assert t.encode(s) == ours.encode(s)
    t.close()
    del meta["tokenizer.ggml.tokens"]
    rlh.write_gguf(p, meta, [])
    with rlh.Gguf(p) as g:
        with pytest.raises(rlh.RlhError) as e:
            rlh.Tokenizer(gguf=g)
    assert e.value.code == rlh.RLH_EFORMAT


def test_invalid_utf8_input_is_refused(bare):
    with pytest.raises(rlh.RlhError) as e:
        bare.encode(b"ab\xffcd")
    assert e.value.code == rlh.RLH_EINVAL
