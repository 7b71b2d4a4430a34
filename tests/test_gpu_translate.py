"""Batch.translateOrdered (OrderedOutput.swift:79-115) on the GPU.

Restates OrderedTests.swift:128-158 (groups of documents, truncation, sequential equality)
on the synthetic model.  Its random weights rarely produce an end token, so documents that
must stop are the one-token prompt recorded in tests/golden/eos_prompts.json (its prefill
prediction is an end id; checked live).  The expected output is simulated from scalar
greedy runs of every document (batch == scalar is bitwise, tests/test_gpu_batch.py), the
restated decodeBatch (oracle/sampler.py, pinned by the OrderedTests KATs) with
stopOnTruncation, and OrderedOutput (tests/test_ordered.py).
"""
import json
import os

import pytest

import plamo_hip
from oracle import sampler

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
S = plamo_hip.Segment


@pytest.fixture(scope="module")
def env(model_dir):
    from plamo_hip import synth
    d, _ = model_dir
    with open(os.path.join(ROOT, "tests", "golden", "eos_prompts.json")) as f:
        eos = json.load(f)["eos_prompts"][0][0]
    path, _ = synth.ensure_tokenizer()
    tok = plamo_hip.Tokenizer(path)
    rt = plamo_hip.Runtime(d, 256)
    assert rt.prefill([eos]) in (1, 16), "recorded end-token prompt no longer stops"
    b = plamo_hip.Batch(rt)
    yield rt, b, tok, eos
    b.close()
    tok.close()
    rt.close()


def _predictions(rt, prompt, limit):
    """Scalar greedy predictions (OrderedTests.swift:117-126): the prefill prediction, then one
    per forward, up to the first end id or `limit` emitted tokens."""
    rt.reset()
    preds = [rt.prefill(prompt)]
    while preds[-1] not in (1, 16) and len(preds) <= limit:
        preds.append(rt.forward([preds[-1]]))
    return preds


def _expected(rt, tok, parts, limit):
    inputs, prefixes, tail = plamo_hip.document_plan(parts)
    text, seqs, discarded = [], [], 0
    for start in range(0, len(inputs), 4):
        end = min(start + 4, len(inputs))
        preds = [_predictions(rt, p, limit) for p in inputs[start:end]]
        cursor = [0] * len(preds)
        sink = plamo_hip.OrderedOutput(tok, prefixes[start:end], tail if end == len(inputs) else "", text.append)
        emitted = [0]

        def step(tokens):
            out = []
            for lane, t in enumerate(tokens):
                if t is not None:
                    cursor[lane] += 1
                out.append(preds[lane][min(cursor[lane], len(preds[lane]) - 1)])
            return out

        def emit(lane, i):
            emitted[0] += 1
            sink.append(lane, i)

        res = sampler.decode_batch([p[0] for p in preds], [limit] * len(preds), step, emit=emit,
                                   finish=lambda lane, o: sink.finish(lane, o), stop_on_truncation=True)
        sink.close()
        seqs += res
        discarded += emitted[0] - sum(len(ids) for ids, _ in res)
        if res[-1][1] != "stop":
            break
    return "".join(text), seqs, discarded, sum(len(p) for p in inputs)


def _run(b, tok, parts, limit):
    text = []
    out = b.translate_ordered(parts, tok, limit, text.append)
    return "".join(text), out


def test_groups_of_four_then_a_truncated_document(env):
    # four documents that stop at once fill the first group (no tail: more follow), the fifth
    # runs alone, ends on its length cap and closes the output (the tail is dropped)
    rt, b, tok, eos = env
    prompt = [int(x) for x in range(1024, 1036)]
    parts = [S("  ", []), S("a", [eos]), S("\r\n", []), S("b", [eos]), S("c", [eos]), S("\t", []),
             S("d", [eos]), S("\n\n", []), S("e", prompt), S(" tail", [])]
    want_text, want_seqs, want_discarded, prefilled = _expected(rt, tok, parts, 10)
    text, out = _run(b, tok, parts, 10)
    print(f"  text {text!r}", flush=True)
    assert [r for _, r in want_seqs] == ["stop"] * 4 + ["length"]
    assert text == want_text and text.startswith("  \r\n\n\t\n\n") and not text.endswith(" tail")
    assert out["sequences"] == want_seqs
    assert out["discarded_tokens"] == want_discarded == 0
    assert out["prefilled_input_tokens"] == prefilled == 16
    assert out["gpu_seconds"] > 0 and out["prefill_seconds"] > 0 and out["decode_seconds"] > 0


def test_truncation_inside_a_group_drops_later_lanes(env):
    # lane 0 ends on its cap while lanes 2 and 3 are still generating: only lane 0 is
    # reported, the tokens lanes 2-3 emitted meanwhile are counted as discarded
    rt, b, tok, eos = env
    parts = [S("<0>", []), S("x", list(range(2000, 2009))), S("<1>", []), S("y", [eos]), S("<2>", []),
             S("z", list(range(3000, 3005))), S("<3>", []), S("w", list(range(4000, 4011))), S("<tail>", [])]
    want_text, want_seqs, want_discarded, _ = _expected(rt, tok, parts, 6)
    text, out = _run(b, tok, parts, 6)
    assert text == want_text and text.startswith("<0>") and "<1>" not in text
    assert out["sequences"] == want_seqs and len(want_seqs) == 1 and want_seqs[0][1] == "length"
    assert out["discarded_tokens"] == want_discarded > 0


def test_every_document_stops_and_the_tail_follows(env):
    rt, b, tok, eos = env
    parts = [S("[", []), S("a", [eos]), S("b", [eos]), S("]", [])]
    text, out = _run(b, tok, parts, 8)
    assert text == "[\n]"
    assert out["sequences"] == [([], "stop"), ([], "stop")] and out["discarded_tokens"] == 0


def test_errors_and_cancellation_reset_the_batch(env):
    rt, b, tok, eos = env
    with pytest.raises(plamo_hip.PlamoError, match="No documents to translate"):
        b.translate_ordered([S(" ", [])], tok, 4, lambda s: None)
    for parts, limit in (([S("a", [eos])], 8192), ([S("a", [107520])], 4), ([S("a", [5] * 250)], 8)):
        with pytest.raises(plamo_hip.PlamoError, match="Invalid document tokens or context budget"):
            b.translate_ordered(parts, tok, limit, lambda s: None)

    class Cancelled(Exception):
        pass

    def cancel(s):
        raise Cancelled()

    with pytest.raises(Cancelled):
        b.translate_ordered([S("p", []), S("a", list(range(1024, 1030)))], tok, 4, cancel)
    assert b.positions() == []  # reset after the error
    text, out = _run(b, tok, [S("a", [eos])], 4)  # still usable
    assert out["sequences"] == [([], "stop")] and text == ""
