"""The byte-level BPE tokenizer (cq_tokenizer_*, the reference's
QwenTokenizer, src/tokenizer.cpp) against HuggingFace `tokenizers`, the
library the Qwen2.5 tokenizer is published for: a byte-level BPE trained
here with the Qwen2 pre-tokenizer pattern, written in the exporter's ranks
layout (export_weights.py:328-365), must encode every test string to the same
ids and decode back to the same bytes.  (No Qwen tokenizer file is available
offline; vocabulary ids of a trained BPE follow its merge order, as Qwen's
do, so the reference's lowest-id merge rule and the library's merge ranks
agree.)"""
import json
import random

import pytest

import cuqwen_amd as cq

PATTERN = (r"""(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*"""
           r"""|\s*[\r\n]+|\s+(?!\S)|\s+""")   # src/tokenizer.cpp:86
SPECIALS = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]
CORPUS = ["Hello world! It's a test, isn't it? We'll see; they're here, I'm sure, you'd know.",
          "def f(x):\n    return x**2  # comment\n\tprint('done')\r\n",
          "Numbers 12345 and 3.14159; dates 2024-01-31, ½ ² ٣٤ Ⅻ.",
          "Привет мир, как дела? Ελληνικά γράμματα. עברית וערבית: مرحبا",
          "日本語のテキストです。中文也可以。한국어 문장입니다.",
          "Ünïcödé àccents naïve café façade Straße ǅungla",
          "tabs\tand  spaces   here\n\n\nnewlines  nbsp em　ideo",
          "emoji 😀👍🏽 and symbols ©®™ → ≤ ≥ ∑ ∫ «quotes» “curly”"]


def train_hf_tokenizer():
    """A byte-level BPE trained with the Qwen2 pre-tokenizer pattern, plus the
    chat special tokens (HuggingFace `tokenizers`)."""
    tk = pytest.importorskip("tokenizers")
    from tokenizers import AddedToken, Regex, decoders, models, pre_tokenizers, trainers
    hf = tk.Tokenizer(models.BPE())
    hf.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(PATTERN), behavior="isolated"),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    hf.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=1500, initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    hf.train_from_iterator(CORPUS * 40, trainer)
    hf.add_special_tokens([AddedToken(s, special=True) for s in SPECIALS])
    return hf


def write_ranks(hf, path):
    """The exporter's ranks layout (export_weights.py:354-363)."""
    data = {"vocab": hf.get_vocab(with_added_tokens=False), "special_tokens": {"eos_token": "<|endoftext|>"},
            "added_tokens": {str(hf.token_to_id(s)): s for s in SPECIALS}}
    path.write_text(json.dumps(data, ensure_ascii=False, indent=2), encoding="utf-8")


@pytest.fixture(scope="module")
def pair(tmp_path_factory):
    hf = train_hf_tokenizer()
    path = tmp_path_factory.mktemp("tok") / "qwen25_bpe_ranks.json"
    write_ranks(hf, path)
    ours = cq.Tokenizer(str(path))
    yield ours, hf, path
    ours.free()


def _random_strings(n, seed):
    rng = random.Random(seed)
    pools = ["abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ", "0123456789", " ", "  \t", "\n\r",
             "'", "sStTmMdDrReEvVlL", ".,;:!?()[]{}<>/\\|@#$%^&*-_=+~`\"", "éüñçßøåÆŒ", "привет",
             "日本語中文", "한국어", "😀👍🏽🚀", "  　", "½²٣Ⅻ", "ǅ"]
    out = []
    for _ in range(n):
        k = rng.randint(1, 40)
        s = "".join(rng.choice(rng.choice(pools)) for _ in range(k))
        if rng.random() < 0.15:
            s = s[:rng.randint(0, len(s))] + rng.choice(SPECIALS) + s[rng.randint(0, len(s)):]
        out.append(s)
    return out


def test_encode_matches_hf_tokenizers(pair):
    ours, hf, _ = pair
    cases = CORPUS + ["", " ", "  ", "\n", " \n ", "a\r\nb", "x  y", "'S 'LL 'Re 'VE don't", "'x", "' s",
                      "<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n", "<|endoftext|><|im_end|>",
                      "123456", "  \t\n\t  x", "a  \n  b", "end   ", "  lead", "\t\tword", " 'hello",
                      "a.b,c;d", "x\n\n\ny", " \r\n\r\n ", "ab" * 300, "!!!???\n\n", "3.14 x"]
    cases += _random_strings(3000, 7)
    bad = [(s, ours.encode(s), hf.encode(s).ids) for s in cases if ours.encode(s) != hf.encode(s).ids]
    assert not bad, bad[:3]


def test_decode_round_trips_and_matches_hf(pair):
    ours, hf, _ = pair
    for s in CORPUS + _random_strings(500, 8):
        ids = ours.encode(s)
        # added tokens are not in the vocabulary, so they decode to nothing
        # (src/tokenizer.cpp:210-211), as the library's skip_special_tokens
        plain = s
        for sp in SPECIALS:
            plain = plain.replace(sp, "")
        assert ours.decode(ids) == plain
        assert ours.decode(ids) == hf.decode(ids, skip_special_tokens=True)
    # single-token pieces of a multi-byte character concatenate to it
    ids = ours.encode("😀")
    assert ours.decode_bytes(ids) == "😀".encode("utf-8")


def test_invalid_utf8_is_kept_byte_for_byte(pair):
    ours, _, _ = pair
    raw = b"ok \xff\xfe bytes \xc3( end \xf0\x9f"
    assert ours.decode_bytes(ours.encode(raw)) == raw


def test_special_tokens_and_lookup(pair):
    ours, hf, _ = pair
    for s in SPECIALS:
        assert ours.token_id(s) == hf.token_to_id(s)
        assert ours.encode(s) == [hf.token_to_id(s)]
    assert ours.token_id("<|not_there|>") == -1
    assert ours.vocab_size() == hf.get_vocab_size(with_added_tokens=True)
    # unknown ids decode to nothing (src/tokenizer.cpp:211)
    assert ours.decode([10 ** 6]) == ""


def test_added_tokens_decode_like_the_reference(tmp_path):
    """src/tokenizer.cpp:48-61, :210-217: the decoder holds the vocabulary
    only, so an added token that is not in vocab.json (Qwen's <|im_end|>)
    decodes to nothing, while a vocabulary entry whose text is an added
    token decodes to that text."""
    data = {"vocab": {"a": 0, "b": 1, "<|endoftext|>": 2}, "special_tokens": {},
            "added_tokens": {"2": "<|endoftext|>", "7": "<|im_end|>"}}
    path = tmp_path / "r.json"
    path.write_text(json.dumps(data), encoding="utf-8")
    t = cq.Tokenizer(str(path))
    try:
        assert t.encode("a<|im_end|>b<|endoftext|>") == [0, 7, 1, 2]
        assert t.decode([0, 7, 1]) == "ab"
        assert t.decode([2, 0]) == "<|endoftext|>a"
    finally:
        t.free()


def test_chat_template_known_answer():
    msgs = [("system", "You are helpful."), {"role": "user", "content": "Hi ☺"}]
    assert cq.Tokenizer.apply_chat_template(msgs, True) == (
        "<|im_start|>system\nYou are helpful.<|im_end|>\n<|im_start|>user\nHi ☺<|im_end|>\n"
        "<|im_start|>assistant\n")
    assert cq.Tokenizer.apply_chat_template(msgs[:1], False) == "<|im_start|>system\nYou are helpful.<|im_end|>\n"
    assert cq.Tokenizer.apply_chat_template([], True) == "<|im_start|>assistant\n"


def test_long_text_grows_the_output(pair):
    ours, hf, _ = pair
    s = "word " * 5000 + "日本語" * 1000
    assert ours.encode(s) == hf.encode(s).ids


def test_load_errors(tmp_path):
    with pytest.raises(cq.CuQwenError, match="cannot open"):
        cq.Tokenizer(str(tmp_path / "missing.json"))
    bad = tmp_path / "bad.json"
    bad.write_text('{"vocab": {"a": 1, "b": }', encoding="utf-8")
    with pytest.raises(cq.CuQwenError, match="tokenizer_load"):
        cq.Tokenizer(str(bad))
    novocab = tmp_path / "novocab.json"
    novocab.write_text('{"added_tokens": {"5": "<|x|>"}}', encoding="utf-8")
    with pytest.raises(cq.CuQwenError, match="vocab"):
        cq.Tokenizer(str(novocab))
    # escapes and surrogate pairs in keys
    esc = tmp_path / "esc.json"
    esc.write_text('{"other": [1, {"x": null}, true], "vocab": {"a": 0, "\\u00e9": 1, "\\ud83d\\ude00": 2, '
                   '"q\\"\\\\": 3}}', encoding="utf-8")
    t = cq.Tokenizer(str(esc))
    assert t.token_id("é") == 1 and t.token_id("😀") == 2 and t.token_id('q"\\') == 3
    t.free()


def test_convert_exports_the_ranks_file(pair, tmp_path):
    """export_tokenizer (export_weights.py:328-365) from a HuggingFace
    directory's vocab.json / tokenizer.json / tokenizer_config.json gives a
    file the tokenizer loads to the same encodings."""
    from cuqwen_amd.convert import export_tokenizer
    ours, hf, _ = pair
    d = tmp_path / "hf"
    d.mkdir()
    hf.save(str(d / "tokenizer.json"))
    (d / "vocab.json").write_text(json.dumps(hf.get_vocab(with_added_tokens=False), ensure_ascii=False),
                                  encoding="utf-8")
    (d / "tokenizer_config.json").write_text(json.dumps({"eos_token": "<|endoftext|>", "model_max_length": 32768,
                                                         "additional_special_tokens": ["<|im_start|>", "xx"]}),
                                             encoding="utf-8")
    out = tmp_path / "ranks.json"
    n_vocab, n_added = export_tokenizer(str(d), str(out))
    assert n_added == 3 and n_vocab == hf.get_vocab_size(with_added_tokens=False)
    data = json.loads(out.read_text(encoding="utf-8"))
    assert set(data) == {"vocab", "special_tokens", "added_tokens"}
    t = cq.Tokenizer(str(out))
    for s in CORPUS + ["<|im_start|>user\nhello<|im_end|>\n"]:
        assert t.encode(s) == ours.encode(s)
    t.free()
