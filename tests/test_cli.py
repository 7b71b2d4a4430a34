"""CLI surface (plamo_hip.cli): Options rules, parseIDs, Sampler.repetitionPeriod and
Segment.split, restating Tests/PlamoTests/OrderedTests.swift:87-99,
SegmentTests.swift:7-62 and SamplerTests.swift:31-37 on the synthetic vocabulary
(tokenizer.jsonl is not available offline).  No GPU: only the tokenizer runs."""
import io
import json
import os

import pytest

import plamo_hip
from plamo_hip import cli, synth


@pytest.fixture(scope="module")
def tok():
    path, _ = synth.ensure_tokenizer()
    t = plamo_hip.Tokenizer(path)
    yield t
    t.close()


@pytest.mark.parametrize("args", [
    ["--batch4"], ["--batch4", "--segment-tokens", "64", "--qsa"], ["--batch4", "--segment-tokens", "64", "--mtp"],
    ["--batch4", "--segment-tokens", "64", "--repetition-penalty", "1.1"],
    ["--batch4", "--segment-tokens", "64", "--frequency-penalty", "0.1"],
    ["--batch4", "--segment-tokens", "64", "--no-repeat-ngram", "1"],
    ["--batch4", "--segment-tokens", "64", "--loop-limit", "4"],
    ["--batch4", "--segment-tokens", "64", "--context", "8192"],
    ["--segment-tokens", "0"], ["--segment-tokens", "63"], ["--segment-tokens", "8193"],
    ["--segment-tokens", "64", "--tokenize", "text"], ["--segment-tokens", "64", "--tokens", "1"],
    ["--segment-tokens", "64", "--decode", "1"], ["--segment-tokens", "64", "--dump-logits", "x"],
    ["--stream", "--repeat", "2"], ["--max-tokens", "0"], ["--qsa-budget", "6"], ["--context", "0"],
    ["--repetition-penalty", "0"], ["--repetition-penalty", "nan"], ["--frequency-penalty", "-1"],
    ["--repetition-penalty", "1e39"], ["--frequency-penalty", "3.5e38"], ["--repetition-penalty", "1e-46"],
    ["--repetition-penalty", " 1.1"], ["--repetition-penalty", "1.1x"], ["--frequency-penalty", "1_0"],
    ["--no-repeat-ngram", "65"], ["--loop-limit", "1001"], ["--max-tokens"], ["--bogus", "1"], ["a", "b"],
    ["--mtp", "--loop-limit", "2"], ["--tokens", "1", "text"]])
def test_options_reject(args):
    with pytest.raises(cli.Failure):
        cli.Options(args)


def test_options_accept():
    assert cli.Options(["--batch4", "--segment-tokens", "512", "--stream"]).batch4
    assert not cli.Options([]).batch4
    assert cli.Options(["--segment-tokens", "512", "--stream"]).segment_tokens == 512
    o = cli.Options(["--tokens", "1,2", "--dump-logits", "f", "--max-tokens", "0"])
    assert (o.max_tokens, o.tokens, o.dump) == (0, "1,2", "f")
    o = cli.Options(["--qsa-budget", "64"])
    assert o.qsa and o.qsa_budget == 64
    with pytest.raises(cli.Failure, match="Missing value for --to"):
        cli.Options(["--to"])


def test_penalties_are_swift_floats():
    # Options stores the penalties as Float (Main.swift:18-19,74-75): one rounding to FP32,
    # so a value that rounds to 1 (or 0) is no sampling control and --batch4 accepts it, and
    # the metrics report the FP32 value
    o = cli.Options(["--batch4", "--segment-tokens", "64", "--repetition-penalty", "1.00000001",
                     "--frequency-penalty", "1e-46"])
    assert o.repetition_penalty == 1.0 and o.frequency_penalty == 0.0
    assert cli.Options(["--repetition-penalty", "1.1"]).repetition_penalty == 1.100000023841858
    assert cli.Options(["--frequency-penalty", "0x1.8p-2"]).frequency_penalty == 0.375
    assert cli.Options(["--repetition-penalty", "3.4e38"]).repetition_penalty == 3.3999999521443642e38


def test_parse_ids():
    assert cli.parse_ids("1,2,107519") == [1, 2, 107519]
    for bad in ["", "1,,2", "1,x", "107520", "-1", "1,2,"]:
        with pytest.raises(cli.Failure):
            cli.parse_ids(bad)


def test_repetition_period_known_answers():
    assert cli.repetition_period([7] * 24, 8) == 1
    assert cli.repetition_period([1, 2, 3, 4] * 8, 8) == 4
    assert cli.repetition_period([1, 2, 3, 4, 5, 6, 7, 8], 8) is None
    assert cli.repetition_period([1, 2, 3, 4], 8) is None
    # period 3 needs ceil(24/3) = 8 copies even when repeats = 2; 7 copies are not enough
    assert cli.repetition_period([5, 6, 7] * 7, 2) is None
    assert cli.repetition_period([9] + [5, 6, 7] * 8, 2) == 3


def _check(parts, text, tok, target, limit):
    assert "".join(p.text for p in parts) == text
    for p in parts:
        if p.tokens:
            assert p.tokens == tok.encode(plamo_hip.Tokenizer.prompt(p.text, target), bos=True)
            assert len(p.tokens) <= limit
            assert not cli._is_white(p.text[0]) and not cli._is_white(p.text[-1])


def test_split_documents(tok):
    text = "\tFirst document.\r\n\r\n  第二文書。 \U0001f9eaé Third document.\n  "
    parts = cli.split_segments(text, "ja", 64, tok)
    _check(parts, text, tok, "ja", 64)
    assert [p.text for p in parts if p.tokens] == ["First document.", "第二文書。 \U0001f9eaé",
                                                   "Third document."]
    blank = "\r\n \t" * 3000 + "Hello."
    parts = cli.split_segments(blank, "ja", 64, tok)
    assert "".join(p.text for p in parts) == blank and len(parts) == 2
    assert not parts[0].tokens and parts[1].tokens


@pytest.mark.parametrize("text", ["A short sentence. 次の文です。 " * 120, "\U00020bb7\U0001f9eaé" * 180,
                                  "abcdef" * 250, "会議は明日です。資料はメールで送ります。参加者は十人です。" * 8])
def test_split_bounds_tokens(tok, text):
    parts = cli.split_segments(text, "en", 64, tok)
    _check(parts, text, tok, "en", 64)
    assert sum(1 for p in parts if p.tokens) > 1


def test_split_keeps_short_text_whole(tok):
    # The synthetic vocabulary spells most Latin letters in bytes, so the whole prompt needs
    # more than the reference's 64 tokens; the rule (the last sentence end in the window
    # that fits) is the same at a limit the synthetic prompt fits.
    text = "First sentence. Second sentence."
    n = len(tok.encode(plamo_hip.Tokenizer.prompt(text, "ja"), bos=True))
    assert [p.text for p in cli.split_segments(text, "ja", n, tok)] == [text]
    assert [p.text for p in cli.split_segments(text, "ja", n - 1, tok) if p.tokens] == ["First sentence.",
                                                                                      "Second sentence."]


def test_sentence_ends_stand_in():
    g = list("Pi is 3.14. Next!  「はい。」次")
    ends = cli._sentence_ends(g)
    assert ["".join(g[:e]) for e in ends] == ["Pi is 3.14.", "Pi is 3.14. Next!", "Pi is 3.14. Next!  「はい。」",
                                             "".join(g)]


@pytest.mark.parametrize("text,target,limit", [("", "en", 64), (" \t\r\n", "en", 64), ("safe\n<|plamo:tag|>", "en", 64),
                                               ("a\uee00b", "en", 64), ("text", "invalid", 64),
                                               ("text", "en", 0), ("a" + "\u0301" * 800, "en", 64)])
def test_split_rejects(tok, text, target, limit):
    with pytest.raises(Exception):
        cli.split_segments(text, target, limit, tok)


def test_tokenize_and_decode_commands(tok, tmp_path):
    path, _ = synth.ensure_tokenizer()
    os.symlink(path, tmp_path / "tokenizer.jsonl")
    out = io.StringIO()
    cli.execute(["--model", str(tmp_path), "--tokenize", "abc 日本語"], None, out, io.StringIO())
    ids = json.loads(out.getvalue())
    assert ids == tok.encode("abc 日本語")
    out = io.StringIO()
    cli.execute(["--model", str(tmp_path), "--decode", ",".join(map(str, ids))], None, out, io.StringIO())
    assert out.getvalue() == "abc 日本語\n"
