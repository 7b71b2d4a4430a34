"""OrderedOutput (OrderedOutput.swift:24-67) through the native library.

The cases restate Tests/PlamoTests/OrderedTests.swift:9-115.  Those tests use the original
vocabulary only for its byte tokens (ASCII byte b at id 384 + b, byte b >= 128 at id b), which
the synthetic vocabulary of test_tokenizer reproduces, so their expected outputs carry over
unchanged.
"""
import os
import random
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path[:0] = [ROOT, os.path.join(ROOT, "plamo3-0.8b-runtime_amd")]

import test_tokenizer as tt  # noqa: E402


class Cancelled(Exception):
    pass


@pytest.fixture(scope="module")
def tok(tmp_path_factory):
    import plamo_hip
    p = tmp_path_factory.mktemp("ord") / "tokenizer.jsonl"
    tt._write(p, tt._records())
    return plamo_hip.Tokenizer(str(p))


def _bytes(text):  # OrderedTests.swift:7
    return [b + 384 if b < 128 else b for b in text.encode()]


def _simulate(tok, texts, limits, prefixes, tail=""):  # OrderedTests.swift:9-23
    import plamo_hip
    source = [_bytes(t) for t in texts]
    out, cursor, calls, seen = [], [0] * len(texts), [], []
    sink = plamo_hip.OrderedOutput(tok, prefixes, tail, out.append)

    def nxt():
        return [source[i][cursor[i]] if cursor[i] < len(source[i]) else (1 if i % 2 == 0 else 16)
                for i in range(len(source))]

    def step(tokens):
        calls.append(list(tokens))
        seen.append("".join(out))
        for lane, t in enumerate(tokens):
            if t is not None:
                assert t == source[lane][cursor[lane]]
                cursor[lane] += 1
        return nxt()

    results = plamo_hip.decode_batch(nxt(), limits, step, emit=sink.append, finish=sink.finish,
                                     stop_on_truncation=True)
    return "".join(out), results, calls, seen


def test_future_eos_and_utf8_stay_in_document_order(tok):
    text, outputs, _, seen = _simulate(tok, ["AAA", "B", "あ", ""], [20] * 4, ["  ", "\r\n\r\n", "\t", "\n"],
                                       "\r\n ")
    assert text == "  AAA\r\n\r\nB\tあ\n\r\n "
    assert [r for _, r in outputs] == ["stop"] * 4
    assert seen == ["  A", "  AA", "  AAA"]
    assert tok.decode(outputs[2][0]) == "あ"


def test_later_truncation_keeps_earlier_document_and_drops_future(tok):
    text, outputs, calls, _ = _simulate(tok, ["AAA", "BBBB", "C", "DDDD"], [20, 2, 20, 20],
                                        ["<0>", "<1>", "<2>", "<3>"], "<tail>")
    assert text == "<0>AAA<1>BB"
    assert [r for _, r in outputs] == ["stop", "length"]
    assert [ids for ids, _ in outputs] == [_bytes("AAA"), _bytes("BB")]
    assert calls[0] == [449, 450, 451, 452]
    assert all(c[1] is None and c[2] is None and c[3] is None for c in calls[1:])
    early = _simulate(tok, ["AAAA", "BBBB", "CCCC", "D"], [2, 20, 1, 20], ["", "<1>", "<2>", "<3>"], "<tail>")
    assert early[0] == "AA" and [r for _, r in early[1]] == ["length"]
    zero = _simulate(tok, ["A", "B"], [0, 20], ["prefix", "later"], "tail")
    assert zero[0] == "prefix" and zero[2] == []


def test_incomplete_future_utf8_and_finish_cancellation(tok):
    import plamo_hip
    out = []
    sink = plamo_hip.OrderedOutput(tok, ["", "\n"], "tail", out.append)
    sink.append(1, 227)
    sink.finish(1, ([227], "stop"))
    assert "".join(out) == ""
    sink.append(0, 449)
    sink.finish(0, ([449], "stop"))
    assert "".join(out) == "A\n�tail"

    def cancel(_):
        raise Cancelled()

    steps = []
    cancelled = plamo_hip.OrderedOutput(tok, ["", "next"], "", cancel)
    with pytest.raises(Cancelled):
        plamo_hip.decode_batch([1, 450], [20, 20], lambda t: steps.append(t) or [1, 16], emit=cancelled.append,
                               finish=cancelled.finish, stop_on_truncation=True)
    assert steps == []


def test_cancellation_and_invalid_output_events(tok):
    import plamo_hip
    from plamo_hip.native import PlamoError
    out, steps = [], []

    def emit(text):
        out.append(text)
        raise Cancelled()

    sink = plamo_hip.OrderedOutput(tok, ["", "next"], "tail", emit)
    with pytest.raises(Cancelled):
        plamo_hip.decode_batch([449, 450], [20, 20], lambda t: steps.append(t) or [1, 16], emit=sink.append,
                               finish=sink.finish, stop_on_truncation=True)
    assert "".join(out) == "A" and steps == []
    valid = plamo_hip.OrderedOutput(tok, [""], "", lambda _: None)
    with pytest.raises(PlamoError, match="Output after document finish"):
        valid.append(1, 449)
    with pytest.raises(PlamoError, match="Token ID out of range"):
        valid.append(0, 107520)
    valid.finish(0, ([], "stop"))
    with pytest.raises(PlamoError, match="Output after document finish"):
        valid.append(0, 449)
    with pytest.raises(PlamoError, match="Invalid document finish"):
        valid.finish(0, ([], "stop"))
    with pytest.raises(PlamoError, match="Expected one to four output prefixes"):
        plamo_hip.OrderedOutput(tok, [], "", lambda _: None)


def test_emitted_text_is_the_repaired_decode(tok):
    # a single document streams everything it is given; its text is the U+FFFD-repaired
    # decode of all bytes, as Swift's String(decoding:as:UTF8.self) repairs each chunk
    import plamo_hip
    rng = random.Random(5)
    for _ in range(300):
        ids = [rng.choice([128 + rng.randrange(128), 384 + rng.randrange(128), rng.randrange(20, 2000)])
               for _ in range(rng.randint(0, 16))]
        out = []
        sink = plamo_hip.OrderedOutput(tok, [""], "", out.append)
        for i in ids:
            sink.append(0, i)
        sink.finish(0, (ids, "stop"))
        assert "".join(out) == tok.decode_bytes(ids).decode("utf-8", errors="replace"), ids


def test_plan_preserves_whitespace_and_adjacent_chunk_boundaries():
    # OrderedTests.swift:52-63
    import plamo_hip
    S = plamo_hip.Segment
    parts = [S("\t", []), S("source A", [449]), S("\r\n", []), S(" \n", []), S("source B", [450]),
             S("source C", [451]), S("\n\t", [])]
    inputs, prefixes, tail = plamo_hip.document_plan(parts)
    assert inputs == [[449], [450], [451]]
    assert prefixes == ["\t", "\r\n \n", "\n"]
    assert tail == "\n\t"
    for bad in ([], [S(" \n", [])]):
        with pytest.raises(plamo_hip.PlamoError, match="No documents to translate"):
            plamo_hip.document_plan(bad)


def test_plan_against_restatement():
    # DocumentPlan (OrderedOutput.swift:3-21) restated in a few lines, on random segment lists:
    # documents keep their order and tokens, every whitespace run lands in exactly one prefix
    # or the tail, and adjacent documents are separated by "\n"
    import plamo_hip
    rng = random.Random(3)
    for _ in range(300):
        parts = []
        for _ in range(rng.randint(1, 9)):
            if rng.random() < 0.5:
                parts.append(plamo_hip.Segment(rng.choice(["", " ", "\n", "\r\n", "\t \n", "あ"]), []))
            else:
                parts.append(plamo_hip.Segment("doc", [rng.randint(0, 107519) for _ in range(rng.randint(1, 4))]))
        want_inputs, want_prefixes, pending = [], [], ""
        for p in parts:
            if not p.tokens:
                pending += p.text
            else:
                want_prefixes.append("\n" if want_inputs and not pending else pending)
                want_inputs.append(list(p.tokens))
                pending = ""
        if not want_inputs:
            with pytest.raises(plamo_hip.PlamoError):
                plamo_hip.document_plan(parts)
            continue
        assert plamo_hip.document_plan(parts) == (want_inputs, want_prefixes, pending)
