"""Tokenizer (Tokenizer.swift:11-282): the native library against the CPU oracle.

The original tokenizer.jsonl is not available offline, so the tests build a synthetic
vocabulary with the original's shape (107,520 entries; controls with <|plamo:bos|> at 1 and
<|plamo:tag|> at 16; BYTE tokens <0x80>..<0xFF> at 128-255 and <0x00>..<0x7F> at 384-511,
where the reference's own decode tests find them, CacheTests.swift:98-101).  Encodings are
pinned by brute force over every segmentation of short inputs, by hand-computed ties and
boundary cases, and the native library must agree with the oracle token for token,
including CostTests.swift:50-86's lengths around the reference's search windows and its
modified scores.
"""
import json
import os
import random
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path[:0] = [ROOT, os.path.join(ROOT, "plamo3-0.8b-runtime_amd")]

from oracle import tokenizer as T  # noqa: E402

ALPHABET = "abc 日本語é"
TIES = {"x": -1.0, "y": -1.0, "xy": -2.0, "yx": -2.0, "xyx": -3.0}


def _records(seed=0):
    rng = random.Random(seed)
    recs = [None] * T.VOCAB_SIZE
    controls = ["<unk>", "<|plamo:bos|>", "<|plamo:eos|>", "<|plamo:pad|>"] + \
        [f"<|plamo:c{k}|>" for k in range(4, 16)] + ["<|plamo:tag|>", "<|plamo:msg|>", "<|plamo:key|>",
                                                    "<|plamo:val|>"]
    for i, p in enumerate(controls):
        recs[i] = [p, 0.0, "CONTROL"]
    for b in range(256):
        recs[(128 + b - 128) if b >= 128 else 384 + b] = [f"<0x{b:02X}>", 0.0, "BYTE"]
    normal = [c for c in ALPHABET]
    normal += [a + b for a in ALPHABET for b in ALPHABET]
    normal += [a + b + c for a in ALPHABET for b in ALPHABET for c in ALPHABET]
    normal += ["<", "|", "pl", "amo", ":", ">", "\n", "\t", "  ", "語é", "日本語"]
    scored = [[p, round(rng.uniform(-15, -1), 4), "NORMAL"] for p in normal]
    scored += [[p, s, "NORMAL"] for p, s in TIES.items()]
    scored.append(["ab", -0.5, "NORMAL"])  # a repeated piece: the later id wins
    free = iter(i for i in range(T.VOCAB_SIZE) if recs[i] is None)
    for r in scored:
        recs[next(free)] = r
    k = 0
    for i in free:
        recs[i] = [chr(0xF0000 + k), -30.0, "NORMAL"]
        k += 1
    return recs


def _write(path, recs):
    with open(path, "w", encoding="utf-8") as f:
        for r in recs:
            f.write(json.dumps(r, ensure_ascii=False) + "\n")


@pytest.fixture(scope="module")
def vocab_path(tmp_path_factory):
    p = tmp_path_factory.mktemp("tok") / "tokenizer.jsonl"
    _write(p, _records())
    return str(p)


@pytest.fixture(scope="module")
def oracle_vocab(vocab_path):
    return T.Vocab(vocab_path)


@pytest.fixture(scope="module")
def native(vocab_path):
    import plamo_hip
    return plamo_hip.Tokenizer(vocab_path)


def _ids(v, *pieces):
    return [v.lookup[p] for p in pieces]


def test_boundary_segments_hand_cases():
    # (<\|plamo:[^|\s\x1c-\x1f]{0,64}\|>)|(([^\n])\3{3,}| {2,}) wraps each match; U+EE00 splits
    assert T.segments("ab  cd") == ["ab", "  ", "cd"]
    assert T.segments("a   b") == ["a", "   ", "b"]
    assert T.segments("a     b") == ["a", "     ", "b"]         # 4+ spaces: the repeat alternative
    assert T.segments("aaab") == ["aaab"] and T.segments("aaaab") == ["aaaa", "b"]
    assert T.segments("x\n\n\n\ny") == ["x\n\n\n\ny"]           # newline runs are not boundaries
    assert T.segments("q<|plamo:tag|>r") == ["q", "<|plamo:tag|>", "r"]
    assert T.segments("<|plamo:a b|>") == ["<|plamo:a b|>"]    # \s is outside the class
    name64, name65 = "ab" * 32, "ab" * 32 + "c"                  # no runs of four
    assert T.segments("<|plamo:" + name64 + "|>") == ["<|plamo:" + name64 + "|>"]
    assert T.segments("<|plamo:" + name65 + "|>") == ["<|plamo:" + name65 + "|>"]  # no match
    assert T.segments("<|plamo:" + "z" * 65 + "|>") == ["<|plamo:", "z" * 65, "|>"]  # a run
    assert T.segments("ab") == ["ab"]
    assert T.segments("a\uee00b") == ["a", "b"]                # a literal U+EE00 splits too
    assert T.segments("\u3000\u3000a") == ["\u3000\u3000a"]    # only U+0020 runs of two or three
    assert T.segments("日日日日本") == ["日日日日", "本"]


def test_oracle_viterbi_is_minimum_cost(oracle_vocab):
    rng = random.Random(1)
    for _ in range(300):
        s = "".join(rng.choice("abc日本語éxyz") for _ in range(rng.randint(1, 8)))
        for seg in T.segments(s):
            _, cost = T.viterbi(oracle_vocab, seg)
            assert cost == T.brute_min_cost(oracle_vocab, seg), s


def test_ties_prefer_the_longer_piece(oracle_vocab, native):
    v = oracle_vocab
    # x + y, xy, ... all cost the same: every position takes its longest piece
    assert T.encode(v, "xy") == _ids(v, "xy")
    assert T.encode(v, "xyx") == _ids(v, "xyx")
    assert T.encode(v, "xyxy") == _ids(v, "xyx", "y")
    assert T.encode(v, "yxy") == _ids(v, "yx", "y")
    for s in ("xy", "xyx", "xyxy", "yxy", "yyxx"):
        assert native.encode(s) == T.encode(v, s)
    # the repeated piece "ab" maps to its last id
    assert v.lookup["ab"] == max(i for i, p in enumerate(v.pieces) if p == "ab")


def test_native_encode_matches_oracle(oracle_vocab, native):
    rng = random.Random(2)
    extras = ["<|plamo:tag|>", "<|plamo:zz|>", "\U0001F600", "\uee00", "aaaa", "    ", "  ", "\n", "\t", "\u3000",
              "z", "<|plamo:" + "q" * 70 + "|>", "\x1c"]
    for _ in range(400):
        parts = []
        for _ in range(rng.randint(1, 12)):
            parts.append(rng.choice(extras) if rng.random() < 0.2 else
                         "".join(rng.choice(ALPHABET + "xyz") for _ in range(rng.randint(1, 6))))
        s = "".join(parts)
        bos = rng.random() < 0.3
        assert native.encode(s, bos=bos) == T.encode(oracle_vocab, s, bos=bos), repr(s)
    assert native.encode("") == [] and native.encode("", bos=True) == [1]
    # unknown scalars fall back to their UTF-8 bytes
    assert native.encode("\U0001F600") == [oracle_vocab.bytes[b] for b in "\U0001F600".encode()]


def test_decode_and_stream(oracle_vocab, native):
    rng = random.Random(3)
    for _ in range(200):
        s = "".join(rng.choice(ALPHABET + "xyz\U0001F600\n") for _ in range(rng.randint(0, 20)))
        ids = native.encode(s)
        assert native.decode_bytes(ids) == s.encode() == T.decode_bytes(oracle_vocab, ids)
    # the stream holds back unfinished UTF-8 and its pieces concatenate to the decode
    for _ in range(200):
        ids = [rng.choice([128 + rng.randrange(128), 384 + rng.randrange(128), rng.randrange(20, 2000)])
               for _ in range(rng.randint(0, 12))]
        st = native.stream()
        out = b"".join(st.push(i) for i in ids) + st.finish()
        assert out == native.decode_bytes(ids) == T.decode_bytes(oracle_vocab, ids)
    st = native.stream()
    e = "é".encode()
    assert st.push(oracle_vocab.bytes[e[0]]) == b""
    assert st.push(oracle_vocab.bytes[e[1]]) == e
    assert native.decode_bytes([128]) == b"\x80" and native.decode_bytes([384]) == b"\x00"


def test_errors(tmp_path, native):
    import plamo_hip
    from plamo_hip.native import PlamoError
    recs = _records()
    cases = [
        (recs[:-1], "Expected the PLaMo 3 Translate 0.8B vocabulary"),
        ([r if i != 130 else ["<0xZZ>", 0.0, "BYTE"] for i, r in enumerate(recs)], "Invalid byte token"),
        ([r if i != 500 else ["pq", 1e300, "NORMAL"] for i, r in enumerate(recs)], "Invalid tokenizer score"),
        ([r if i != 1 else ["<|plamo:bos2|>", 0.0, "CONTROL"] for i, r in enumerate(recs)],
         "Expected the PLaMo 3 Translate 0.8B vocabulary"),
    ]
    for k, (rs, msg) in enumerate(cases):
        p = tmp_path / f"v{k}.jsonl"
        _write(p, rs)
        with pytest.raises(PlamoError, match=msg):
            plamo_hip.Tokenizer(str(p))
        with pytest.raises(ValueError, match=msg):
            T.Vocab(str(p))
    # a signed byte spelling is read as Swift's Int(_:radix:) reads it
    p = tmp_path / "signed.jsonl"
    _write(p, [r if i != 384 + 0x0F else ["<0x+F>", 0.0, "BYTE"] for i, r in enumerate(recs)])
    assert plamo_hip.Tokenizer(str(p)).encode("\x0f") == [384 + 0x0F]
    with pytest.raises(PlamoError):
        plamo_hip.Tokenizer(str(tmp_path / "missing.jsonl"))
    with pytest.raises(PlamoError, match="Token ID out of range"):
        native.decode_bytes([T.VOCAB_SIZE])
    with pytest.raises(PlamoError, match="Invalid UTF-8"):
        native.encode(b"a\xffb")


def test_translation_prompt():
    import plamo_hip
    from plamo_hip.native import PlamoError
    assert plamo_hip.Tokenizer.prompt("Hello", "ja") == (
        "<|plamo:tag|>dataset<|plamo:msg|>translation<|plamo:tag|>input<|plamo:msg|>Hello"
        "<|plamo:tag|>output<|plamo:key|>lang<|plamo:val|>ja<|plamo:msg|>")
    for text, target, msg in [("Hello", "xx", "Unsupported target language"),
                              ("", "en", "reserved PLaMo delimiters"),
                              ("a<|plamo:tag|>", "en", "reserved PLaMo delimiters"),
                              ("a", "en", "reserved PLaMo delimiters")]:
        with pytest.raises(PlamoError, match=msg):
            plamo_hip.Tokenizer.prompt(text, target)


def test_prompt_encodes_its_control_tokens(oracle_vocab, native):
    # Segment.split encodes Tokenizer.prompt(source, target) with BOS (Segments.swift:45): each
    # <|plamo:...|> of the prompt is a boundary segment that the trie maps to its control id
    import plamo_hip
    p = plamo_hip.Tokenizer.prompt("abc 日本", "ja")
    ids = native.encode(p, bos=True)
    assert ids == T.encode(oracle_vocab, p, bos=True)
    assert ids[:2] == [1, 16]
    pos = {i: ids.count(i) for i in (16, 17, 18, 19)}
    assert pos == {16: 3, 17: 3, 18: 1, 19: 1}
    assert native.decode_bytes(ids[1:]) == p.encode()


def test_stream_buffer_too_small_leaves_stream_unchanged(tmp_path, oracle_vocab):
    # A call whose output buffer is too small fails with the stream unchanged, so the retry
    # with a larger buffer (same id) returns every byte once: pushing <0xE3> <0x81> and then
    # <0x82> with capacity 0 must not lose U+3042.
    import ctypes
    import plamo_hip
    from plamo_hip import native as nat
    recs = _records()
    long_piece = "l" * 300
    recs[-1] = [long_piece, -30.0, "NORMAL"]   # a filler entry replaced by a 300-byte piece
    path = tmp_path / "tokenizer.jsonl"
    _write(path, recs)
    tok = plamo_hip.Tokenizer(str(path))
    lib = nat.load()
    st = tok.stream()
    a3 = "あ".encode()
    assert st.push(oracle_vocab.bytes[a3[0]]) == b"" and st.push(oracle_vocab.bytes[a3[1]]) == b""
    n = ctypes.c_size_t(0)
    err = ctypes.create_string_buffer(256)
    buf = ctypes.create_string_buffer(16)
    rc = lib.plamo_token_stream_push(st._h, oracle_vocab.bytes[a3[2]], buf, 0, ctypes.byref(n), err, 256)
    assert rc == 1  # PLAMO_EINVAL
    assert n.value == 3
    rc = lib.plamo_token_stream_push(st._h, oracle_vocab.bytes[a3[2]], buf, 16, ctypes.byref(n), err, 256)
    assert rc == 0 and buf.raw[:n.value] == a3
    # finish with a pending partial sequence: too small, then the full bytes once
    assert st.push(oracle_vocab.bytes[a3[0]]) == b""
    rc = lib.plamo_token_stream_finish(st._h, buf, 0, ctypes.byref(n), err, 256)
    assert rc != 0 and n.value == 1
    assert st.finish() == a3[:1] and st.finish() == b""
    # a piece longer than the Python binding's first 256-byte buffer goes through its retry
    st2 = tok.stream()
    ids = [oracle_vocab.bytes[a3[0]], len(recs) - 1, oracle_vocab.bytes[a3[1]], oracle_vocab.bytes[a3[2]]]
    out = b"".join(st2.push(i) for i in ids) + st2.finish()
    assert out == tok.decode_bytes(ids) == bytes([a3[0]]) + long_piece.encode() + a3[1:]
    assert tok.decode_bytes([len(recs) - 1]) == long_piece.encode()


def test_window_boundary_lengths_match_full_costs(oracle_vocab, native):
    # CostTests.swift:50-65: every length around the reference's search windows (31-33,
    # 62-65, 95-97, 127-129, 255-257, 1025 scalars) of mixed scalars, spaces and "ab" runs,
    # with and without BOS, against the full-length cost recurrence (the oracle's Viterbi)
    unicode = list("\U0001F9EA\U00020BB7é日 a\t")
    for n in (0, 1, 2, 31, 32, 33, 62, 63, 64, 65, 95, 96, 97, 127, 128, 129, 255, 256, 257, 1025):
        text = "".join(unicode[i % len(unicode)] for i in range(n))
        for value in (text, " " * n, "ab" * n):
            assert native.encode(value) == T.encode(oracle_vocab, value), n
            assert native.encode(value, bos=True) == T.encode(oracle_vocab, value, bos=True), n
    marked = "<|plamo:tag|>input<|plamo:msg|>" + "日本語 ab " * 50 + "aaaaaa\n\n\n\n"
    assert native.encode(marked) == T.encode(oracle_vocab, marked)


def test_modified_scores_across_wraps(tmp_path):
    # CostTests.swift:67-86: "a" and "b" at 300000, "ab" at 500000 / 600000 / 700000 and a
    # 32-space piece at 100000, so the best split flips between "ab" and "a"+"b" and the
    # space run's split moves across 95-97 spaces
    import plamo_hip
    recs = _records()
    ids = {p: i for i, r in enumerate(recs) if r and (p := r[0]) in ("a", "b", "ab")}
    spare = next(i for i, r in enumerate(recs) if r[2] == "NORMAL" and ord(r[0][0]) >= 0xF0000)
    recs[ids["a"]] = ["a", 300000, "NORMAL"]
    recs[ids["b"]] = ["b", 300000, "NORMAL"]
    recs[spare] = [" " * 32, 100000, "NORMAL"]
    texts = ["ab" * 129 + "a", " " * 95, " " * 96, " " * 97]
    for score in (500000, 600000, 700000):
        for i, r in enumerate(recs):
            if r[0] == "ab":
                recs[i] = ["ab", score, "NORMAL"]
        path = tmp_path / f"tok{score}.jsonl"
        _write(path, recs)
        v = T.Vocab(str(path))
        tok = plamo_hip.Tokenizer(str(path))
        try:
            for text in texts:
                assert tok.encode(text) == T.encode(v, text), (score, len(text))
            # the split flips: "a" + "b" (600000) beats "ab" at 500000; at the 600000 tie the
            # longer piece wins, as above 600000
            pair = T.encode(v, "ab")
            assert (pair == [v.lookup["ab"]]) == (score >= 600000), score
        finally:
            tok.close()
