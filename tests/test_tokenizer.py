"""The byte-level BPE tokenizer (include/lcr_tokenizer.h), on the CPU.

  - the reference's own cases (tests/test_tokenizer.cpp:86-253): the Llama 3
    split of 28 strings, the byte-level alphabet, merges with and without
    ignore_merges on a synthetic tokenizer.json, added tokens, round trips
    and the rejections of other tokenizers;
  - against Hugging Face's tokenizers library (an independent implementation
    of the same format): its Split pre-tokenizer with the Llama 3 pattern on
    seeded strings mixing letters of several scripts, digits, white space of
    every kind, line breaks, contractions, punctuation and symbols; and full
    encodes and decodes with byte-level BPE models trained here on a seeded
    corpus, with ignore_merges on and off and special tokens in the text.
"""

import json
import random
import time

import pytest

LLAMA3_PATTERN = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}{1,3}| ?[^\s\p{L}\p{N}]+[\r\n]*|"
                  r"\s*[\r\n]+|\s+(?!\S)|\s+")


def split(lcr, text):
    return [p.decode("utf-8", errors="surrogateescape") for p in lcr.split_pretokens(text)]


# tests/test_tokenizer.cpp:86-130
SPLIT_CASES = [
    ("", []),
    ("Hello world", ["Hello", " world"]),
    ("Hello, world!", ["Hello", ",", " world", "!"]),
    ("don't", ["don", "'t"]),
    ("DON'T", ["DON", "'T"]),
    ("they're", ["they", "'re"]),
    ("I'll've", ["I", "'ll", "'ve"]),
    ("1234567", ["123", "456", "7"]),
    ("v2.0", ["v", "2", ".", "0"]),
    ("a  b", ["a", " ", " b"]),
    ("  hello", [" ", " hello"]),
    ("  \n", ["  \n"]),
    ("a\n\nb", ["a", "\n\n", "b"]),
    ("a \n b", ["a", " \n", " b"]),
    ("a   ", ["a", "   "]),
    ("()", ["()"]),
    (" (x)", [" (", "x", ")"]),
    ("...", ["..."]),
    ("café", ["café"]),
    ("日本語", ["日本語"]),
    ("hi 🙂", ["hi", " 🙂"]),
    ("'x", ["'x"]),
    (" 's", [" '", "s"]),
]


@pytest.mark.parametrize("text,want", SPLIT_CASES)
def test_split_reference_cases(lcr, text, want):
    got = split(lcr, text)
    assert got == want
    assert "".join(got) == text


def test_byte_level_alphabet(lcr):
    tok = lcr.Tokenizer(json_text=synthetic_tokenizer_json(False))
    all_bytes = bytes(range(256))
    ids = tok.encode(all_bytes, parse_special=False)
    assert tok.decode(ids) == all_bytes
    # ' ' is U+0120 and '\n' U+010A in the vocabulary (ids of the one-byte pieces)
    assert tok.token_to_id("Ġ") == ord(" ")
    assert tok.token_to_id("Ċ") == ord("\n")
    assert tok.token_to_id("!") == ord("!")


def byte_char(b):
    """GPT-2 byte-level character of byte b, written from its definition."""
    printable = list(range(0x21, 0x7F)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    if b in printable:
        return chr(b)
    return chr(256 + [x for x in range(256) if x not in printable].index(b))


def synthetic_tokenizer_json(ignore_merges: bool, pattern: str = LLAMA3_PATTERN) -> str:
    """The reference's in-memory test tokenizer (tests/test_tokenizer.cpp:34-66):
    ids 0..255 are the bytes, 256 "ab" and 257 " ab" are reachable by the two
    merges, 258 "xyz" is in the vocabulary but no merge builds it, and three
    added tokens."""
    vocab = {byte_char(b): b for b in range(256)}
    vocab["ab"] = 256
    vocab[byte_char(32) + "ab"] = 257
    vocab["xyz"] = 258
    doc = {
        "version": "1.0",
        "added_tokens": [{"id": 300, "content": "<|eot|>", "special": True},
                         {"id": 301, "content": "<|begin_of_text|>", "special": True},
                         {"id": 302, "content": "<|long_special_token|>", "special": True}],
        "pre_tokenizer": {"type": "Sequence", "pretokenizers": [
            {"type": "Split", "pattern": {"Regex": pattern}, "behavior": "Isolated", "invert": False},
            {"type": "ByteLevel", "add_prefix_space": False, "trim_offsets": True, "use_regex": False}]},
        "decoder": {"type": "ByteLevel"},
        "model": {"type": "BPE", "ignore_merges": ignore_merges, "vocab": vocab,
                  "merges": ["a b", byte_char(32) + " ab"]},
    }
    return json.dumps(doc)


def test_bpe_merges(lcr):
    """tests/test_tokenizer.cpp:141-168."""
    tok = lcr.Tokenizer(json_text=synthetic_tokenizer_json(False))
    assert tok.vocab_size == 303
    assert tok.bos_id == 301
    assert tok.encode("ab") == [256]
    assert tok.encode("ab ab") == [256, 257]
    assert tok.encode("qr") == [ord("q"), ord("r")]
    assert tok.encode("xyz") == [ord("x"), ord("y"), ord("z")]
    ign = lcr.Tokenizer(json_text=synthetic_tokenizer_json(True))
    assert ign.encode("xyz") == [258]
    assert ign.encode("ab ab") == [256, 257]
    assert ign.encode("abq") == [256, ord("q")]


def test_added_tokens(lcr):
    """tests/test_tokenizer.cpp:170-194."""
    tok = lcr.Tokenizer(json_text=synthetic_tokenizer_json(True))
    assert tok.encode("hi<|eot|>", False, True) == [ord("h"), ord("i"), 300]
    literal = tok.encode("hi<|eot|>", False, False)
    assert len(literal) > 3 and 300 not in literal
    assert tok.encode("<|long_special_token|>") == [302]
    assert tok.encode("ab", True, True) == [301, 256]
    assert tok.encode("<|eot|>ab ab<|eot|>", False, True) == [300, 256, 257, 300]


def test_decode_round_trip(lcr):
    """tests/test_tokenizer.cpp:196-228."""
    tok = lcr.Tokenizer(json_text=synthetic_tokenizer_json(True))
    samples = ["", "ab ab", "Hello, world!", "don't stop\n\n  indented", "café 日本語 🙂",
               "tabs\tand\rcarriage returns"]
    raw_samples = [s.encode() for s in samples] + [b"nul\x00inside", b"\xff\xfe raw bytes that are not utf-8"]
    for raw in raw_samples:
        ids = tok.encode(raw)
        assert tok.decode(ids) == raw
        assert b"".join(tok.decode([i]) for i in ids) == raw
    assert tok.decode([300]) == b"<|eot|>"
    assert tok.decode([300], skip_special=True) == b""
    assert tok.is_special(300) and not tok.is_special(ord("a"))
    assert tok.token_to_id("<|eot|>") == 300
    assert tok.token_to_id("ab") == 256
    assert tok.token_to_id("no such token") == -1


def test_rejects_incompatible_tokenizers(lcr):
    """tests/test_tokenizer.cpp:230-253."""
    with pytest.raises(lcr.LcrError, match="pretokenizer pattern this runtime does not implement"):
        lcr.Tokenizer(json_text=synthetic_tokenizer_json(True, r"\w+|[^\w\s]+"))
    with pytest.raises(lcr.LcrError, match="only implements byte-level BPE"):
        lcr.Tokenizer(json_text=json.dumps({"model": {"type": "Unigram", "vocab": []}}))
    with pytest.raises(lcr.LcrError, match="no Split pretokenizer"):
        lcr.Tokenizer(json_text=json.dumps({"model": {"type": "BPE", "vocab": {"a": 0}, "merges": []}}))


# ---------------------------------------------------------------------------
# against Hugging Face tokenizers
# ---------------------------------------------------------------------------

ALPHABET = (
    list("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ") * 3
    + list("0123456789") * 2
    + [" "] * 12 + ["\n"] * 3 + ["\r", "\t", " ", "　", " ", " ", "\x0b", "\x0c", "\x85"]
    + list("'''''") + list(".,;:!?()[]{}<>-_=+*/\\|\"#$%&@^`~")
    + list("éüßçñøåÆŒЖжЯщΩλπ") + list("日本語中文한국어") + list("٠١٢٣") + list("ⅣⅫ½²³")
    + ["🙂", "🚀", "✓", "€", "£", "©", "°", "​", "́", "א", "ا"]
    + ["'s", "'t", "'re", "'ve", "'m", "'ll", "'d", "'S", "'RE", "'Ll"]
)


def random_text(r, n):
    return "".join(r.choice(ALPHABET) for _ in range(n))


def hf_split(text):
    from tokenizers import Regex, pre_tokenizers
    pt = pre_tokenizers.Split(Regex(LLAMA3_PATTERN), behavior="isolated", invert=False)
    return [piece for piece, _ in pt.pre_tokenize_str(text)]


def test_split_matches_huggingface(lcr):
    pytest.importorskip("tokenizers")
    r = random.Random(5)
    texts = [random_text(r, r.randint(1, 60)) for _ in range(1500)]
    texts += ["\n\n\n", "   \n\n  \t", "x\r\n\r\ny", "word  　 next", "a b", "12345 67 8",
              "it's DON'T I'D we'Ve", "''s'", "\t\tindent", "end with space ", "  "]
    for text in texts:
        assert split(lcr, text) == hf_split(text), repr(text)


def corpus(seed, n_lines):
    r = random.Random(seed)
    words = ["the", "quick", "brown", "fox", "jumps", "over", "lazy", "dog", "don't", "it's", "we'll", "café",
             "naïve", "日本", "語", "1234", "3.14159", "hello", "world", "tokenizer", "byte", "level", "merge",
             "🙂", "(x)", "[y]", "a+b=c", "\t", "  ", "\n"]
    return [" ".join(r.choice(words) for _ in range(r.randint(3, 18))) for _ in range(n_lines)]


SPECIALS = ["<|begin_of_text|>", "<|end_of_text|>", "<|start_header_id|>", "<|end_header_id|>", "<|eot_id|>"]


def trained_tokenizer(vocab_size: int, ignore_merges: bool):
    from tokenizers import Regex, Tokenizer, decoders, models, pre_tokenizers, trainers
    tok = Tokenizer(models.BPE(ignore_merges=ignore_merges))
    tok.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(LLAMA3_PATTERN), behavior="isolated", invert=False),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=vocab_size, special_tokens=SPECIALS, show_progress=False,
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    tok.train_from_iterator(corpus(11, 3000), trainer=trainer)
    return tok


@pytest.mark.parametrize("ignore_merges", [False, True])
def test_encode_matches_huggingface(lcr, ignore_merges):
    pytest.importorskip("tokenizers")
    hf = trained_tokenizer(1200, ignore_merges)
    ours = lcr.Tokenizer(json_text=hf.to_str())
    assert ours.vocab_size == hf.get_vocab_size()
    assert ours.bos_id == hf.token_to_id("<|begin_of_text|>")
    r = random.Random(17)
    texts = corpus(23, 400) + [random_text(r, r.randint(1, 80)) for _ in range(400)]
    texts += ["<|begin_of_text|><|start_header_id|>user<|end_header_id|>\n\nHello there<|eot_id|>",
              "text <|eot_id|>more<|eot_id|><|eot_id|>", "<|not_a_special|>"]
    for text in texts:
        want = hf.encode(text, add_special_tokens=False).ids
        got = ours.encode(text, add_bos=False, parse_special=True)
        assert got == want, repr(text)
        assert ours.decode(got) == text.encode()
        assert ours.decode(got, skip_special=True).decode() == hf.decode(want, skip_special_tokens=True)


def synthetic_llama3_scale_json(vocab_size=128000, seed=5):
    """A byte-level BPE tokenizer.json of Llama 3's size: the GPT-2 byte
    alphabet, then merges of existing pieces (so every merge is valid) up to
    128,000 pieces, 256 special tokens after them, ignore_merges on."""
    r = random.Random(seed)
    bs = list(range(ord("!"), ord("~") + 1)) + list(range(ord("¡"), ord("¬") + 1)) + list(range(ord("®"), ord("ÿ") + 1))
    cs = bs[:]
    n = 0
    for b in range(256):
        if b not in bs:
            bs.append(b)
            cs.append(256 + n)
            n += 1
    pieces = [chr(c) for c in cs]
    vocab = {p: i for i, p in enumerate(pieces)}
    merges = []
    while len(vocab) < vocab_size:
        a = pieces[r.randrange(min(len(pieces), 256 + len(pieces) // 2))]
        b = pieces[r.randrange(min(300, len(pieces)))]
        new = a + b
        if new in vocab or len(new) > 12:
            continue
        vocab[new] = len(vocab)
        pieces.append(new)
        merges.append(f"{a} {b}")
    names = ["<|begin_of_text|>", "<|end_of_text|>"] + [f"<|reserved_special_token_{i}|>" for i in range(254)]
    added = [{"id": vocab_size + i, "content": c, "single_word": False, "lstrip": False, "rstrip": False,
              "normalized": False, "special": True} for i, c in enumerate(names)]
    return json.dumps({
        "version": "1.0", "added_tokens": added, "normalizer": None,
        "pre_tokenizer": {"type": "Sequence", "pretokenizers": [
            {"type": "Split", "pattern": {"Regex": LLAMA3_PATTERN}, "behavior": "Isolated", "invert": False},
            {"type": "ByteLevel", "add_prefix_space": False, "trim_offsets": True, "use_regex": False}]},
        "post_processor": None,
        "decoder": {"type": "ByteLevel", "add_prefix_space": True, "trim_offsets": True, "use_regex": True},
        "model": {"type": "BPE", "dropout": None, "unk_token": None, "continuing_subword_prefix": None,
                  "end_of_word_suffix": None, "fuse_unk": False, "byte_fallback": False, "ignore_merges": True,
                  "vocab": vocab, "merges": merges}})


def test_llama3_scale_tokenizer_matches_huggingface(lcr, tmp_path):
    """At Llama 3's size (128,256 entries, about 128,000 merges, an 8 MB
    file): the file loads in seconds, and 1500 texts and their concatenation
    encode to Hugging Face's ids and decode back to their bytes."""
    pytest.importorskip("tokenizers")
    from tokenizers import Tokenizer as HfTokenizer
    path = tmp_path / "tokenizer.json"
    path.write_text(synthetic_llama3_scale_json())
    t0 = time.perf_counter()
    ours = lcr.Tokenizer(path)
    load_s = time.perf_counter() - t0
    hf = HfTokenizer.from_file(str(path))
    assert ours.vocab_size == hf.get_vocab_size() == 128256
    assert load_s < 10.0, load_s
    r = random.Random(21)
    texts = corpus(31, 1000) + [random_text(r, r.randint(1, 120)) for _ in range(500)]
    for text in texts:
        assert ours.encode(text) == hf.encode(text, add_special_tokens=False).ids, text
    whole = "\n".join(texts)
    ids = ours.encode(whole)
    assert ids == hf.encode(whole, add_special_tokens=False).ids
    assert ours.decode(ids) == whole.encode()
