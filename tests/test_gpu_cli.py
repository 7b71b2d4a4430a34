"""The plamo command (plamo_hip.cli) end to end on the GPU with the synthetic model.

Checks the stderr metrics schema (Main.swift:331-347 top-level keys, 265-273 run keys), that
the command's tokens equal the runtime's own greedy loop, --stream text equal to the plain
text, --dump-logits, the segment pipeline's stop rule (SegmentTests.swift:97-107: a
truncated segment stops the pipeline, and segments that stop on an end id let the next one
run, adjacent ones joined by a newline), and the command run as a fresh process: the
translation alone on stdout and exactly one JSON line on stderr (web/server.ts:22-58 reads
stdout as the translation and parses all of stderr), and BatchCLITests.swift:5-60's
--batch4 against the sequential segment loop."""
import io
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import plamo_hip
from plamo_hip import cli, synth

pytestmark = pytest.mark.gpu

TOP = {"device", "load_seconds", "packed", "qsa", "qsa_budget", "mtp", "repetition_penalty", "frequency_penalty",
       "no_repeat_ngram", "peak_rss_bytes", "physical_footprint_bytes", "peak_physical_footprint_bytes",
       "resident_bytes", "metal_allocated_bytes", "peak_metal_allocated_bytes", "gpu_weight_bytes",
       "auxiliary_weight_bytes", "context", "segment_tokens", "batch4", "runs"}
RUN = {"input_tokens", "output_tokens", "prefill_seconds", "decode_seconds", "decode_tokens_per_second",
       "gpu_seconds", "stop_reason", "output_ids", "mtp_proposed_tokens", "mtp_accepted_tokens",
       "mtp_verifications", "qsa_queries", "qsa_selected_keys", "qsa_dense_keys"}
TEXT = "abc 日本語. cab 語本日."
UNBROKEN = "会議は明日です。資料はメールで送ります。参加者は十人です。" * 8


@pytest.fixture(scope="module")
def model(model_dir, tmp_path_factory):
    d, _ = model_dir
    m = tmp_path_factory.mktemp("cli_model")
    for name in os.listdir(d):
        os.symlink(os.path.join(d, name), m / name)
    if not (m / "tokenizer.jsonl").exists():
        os.symlink(synth.ensure_tokenizer()[0], m / "tokenizer.jsonl")
    return str(m)


def run(model, args, text=None):
    out, err = io.StringIO(), io.StringIO()
    cli.execute(["--model", model] + args + ([text] if text is not None else []), None, out, err)
    return out.getvalue(), json.loads(err.getvalue())


def test_metrics_schema_and_greedy_tokens(model):
    out, m = run(model, ["--max-tokens", "8"], TEXT)
    assert set(m) == TOP and len(m["runs"]) == 1 and set(m["runs"][0]) == RUN
    r = m["runs"][0]
    tok = plamo_hip.Tokenizer(os.path.join(model, "tokenizer.jsonl"))
    prompt = tok.encode(plamo_hip.Tokenizer.prompt(TEXT, "ja"), bos=True)
    with plamo_hip.Runtime(model, 256) as rt:
        ids, reason = rt.generate(prompt, 8)
    assert r["output_ids"] == ids and r["input_tokens"] == len(prompt)
    assert r["stop_reason"] == (reason or "length") and m["context"] == len(prompt) + 8
    assert out == tok.decode(ids) + "\n"
    assert m["gpu_weight_bytes"] > 0 and m["metal_allocated_bytes"] >= m["gpu_weight_bytes"]
    streamed, _ = run(model, ["--max-tokens", "8", "--stream"], TEXT)
    assert streamed == tok.decode(ids)
    tok.close()


def test_dump_logits_prefill_only(model, tmp_path):
    f = str(tmp_path / "logits.f32")
    _, m = run(model, ["--tokens", "1,5,9,300", "--dump-logits", f, "--max-tokens", "0"])
    assert m["runs"][0]["stop_reason"] == "prefill" and m["runs"][0]["output_ids"] == []
    with plamo_hip.Runtime(model, 64) as rt:
        rt.prefill([1, 5, 9, 300])
        want = rt.logits()
    assert np.array_equal(np.fromfile(f, dtype="<f4"), want)


def test_segment_pipeline_and_batch4(model):
    tok = plamo_hip.Tokenizer(os.path.join(model, "tokenizer.jsonl"))
    parts = [p for p in cli.split_segments(UNBROKEN, "en", 64, tok) if p.tokens]
    assert len(parts) > 1
    first, m1 = run(model, ["--stream", "--to", "en", "--max-tokens", "4"], parts[0].text)
    chunked, m = run(model, ["--stream", "--to", "en", "--max-tokens", "4", "--segment-tokens", "64"], UNBROKEN)
    r = m["runs"][0]
    assert r["segments_total"] == len(parts)
    # the first segment runs to its limit (the synthetic model does not stop on these prompts),
    # so the pipeline ends after it
    assert m1["runs"][0]["stop_reason"] == "length"
    assert chunked == first and r["stop_reason"] == "length" and r["segments_completed"] == 0
    assert r["output_ids"] == m1["runs"][0]["output_ids"]
    _, b = run(model, ["--to", "en", "--max-tokens", "4", "--segment-tokens", "64", "--batch4"], UNBROKEN)
    rb = b["runs"][0]
    assert {"prefilled_input_tokens", "discarded_output_tokens", "segments", "segments_total"} <= set(rb)
    assert rb["segments"][0]["output_ids"] == m1["runs"][0]["output_ids"]
    tok.close()


def test_segments_that_stop_let_the_next_run(model, monkeypatch):
    # A segment whose prompt predicts an end id stops with no tokens ("stop"), and the
    # pipeline goes on (Main.swift's segment loop): adjacent text segments are joined by a
    # newline, literal pieces are copied, and the last segment runs to its limit.  The
    # synthetic model stops at once only on the one-token prompt of tests/golden/eos_prompts.json,
    # so the segmenter's output is replaced by segments made of it.
    with open(os.path.join(os.path.dirname(__file__), "golden", "eos_prompts.json")) as f:
        eos = json.load(f)["eos_prompts"][0][0]
    tok = plamo_hip.Tokenizer(os.path.join(model, "tokenizer.jsonl"))
    last = tok.encode(plamo_hip.Tokenizer.prompt("abc 日本語.", "en"), bos=True)
    tok.close()
    parts = [plamo_hip.Segment("x", [eos]), plamo_hip.Segment("y", [eos]), plamo_hip.Segment(" \t", []),
             plamo_hip.Segment("z", last)]
    monkeypatch.setattr(cli, "split_segments", lambda *a: parts)
    _, one = run(model, ["--to", "en", "--max-tokens", "4"], "abc 日本語.")
    assert one["runs"][0]["stop_reason"] == "length"
    out, m = run(model, ["--to", "en", "--max-tokens", "4", "--segment-tokens", "64"], "x y z")
    r = m["runs"][0]
    assert [s["stop_reason"] for s in r["segments"]] == ["stop", "stop", "length"]
    assert r["segments_completed"] == 2 and r["segments_total"] == 3 and r["stop_reason"] == "length"
    assert r["output_ids"] == one["runs"][0]["output_ids"]
    tok = plamo_hip.Tokenizer(os.path.join(model, "tokenizer.jsonl"))
    assert out == "\n" + " \t" + tok.decode(r["output_ids"]) + "\n"
    tok.close()
    out_b, b = run(model, ["--to", "en", "--max-tokens", "4", "--segment-tokens", "64", "--batch4"], "x y z")
    rb = b["runs"][0]
    assert [s["stop_reason"] for s in rb["segments"]] == ["stop", "stop", "length"]
    assert rb["segments_completed"] == 2 and rb["output_ids"] == r["output_ids"] and out_b == out


def test_command_in_a_fresh_process(model):
    # what web/server.ts spawns: a new process, whose first HIP call happens in it
    env = dict(os.environ, PYTHONPATH=os.pathsep.join(
        [os.path.join(os.path.dirname(os.path.dirname(__file__)), "plamo3-0.8b-runtime_amd"),
         os.environ.get("PYTHONPATH", "")]))
    p = subprocess.run([sys.executable, "-m", "plamo_hip.cli", "--model", model, "--max-tokens", "8", TEXT],
                       capture_output=True, env=env, timeout=110)
    assert p.returncode == 0, p.stderr.decode(errors="replace")
    lines = p.stderr.decode().splitlines()
    assert len(lines) == 1, lines
    m = json.loads(lines[0])
    want, wm = run(model, ["--max-tokens", "8"], TEXT)
    assert m["runs"][0]["output_ids"] == wm["runs"][0]["output_ids"]
    assert p.stdout.decode() == want
    bad = subprocess.run([sys.executable, "-m", "plamo_hip.cli", "--model", model, "--repetition-penalty", "0", TEXT],
                         capture_output=True, env=env, timeout=110)
    assert bad.returncode == 1 and bad.stdout == b""
    assert bad.stderr.decode() == "error: Repetition penalty must be a positive finite number\n"


def test_mtp_output_is_the_greedy_sequence(model, model_dir, monkeypatch):
    # --mtp drafts with the adapter and keeps only what a sequential verification pass
    # predicts (Main.swift:254-276), so the output ids are greedy decoding's; the counters
    # follow the loop (every verification proposes at most one draft)
    monkeypatch.setenv("PLAMO_SOURCE_SHA256", model_dir[1])
    out, m = run(model, ["--max-tokens", "12"], TEXT)
    out_mtp, mm = run(model, ["--max-tokens", "12", "--mtp"], TEXT)
    r, rm = m["runs"][0], mm["runs"][0]
    assert rm["output_ids"] == r["output_ids"] and out_mtp == out
    assert mm["mtp"] is True and mm["auxiliary_weight_bytes"] == 2 * (256 * 3072 + 1536 * 256)
    assert rm["mtp_verifications"] >= 1 and 0 <= rm["mtp_accepted_tokens"] <= rm["mtp_proposed_tokens"]
    assert rm["mtp_proposed_tokens"] <= rm["mtp_verifications"]
    # each verification keeps its first candidate plus the accepted drafts; a last single
    # token goes out without one
    assert len(rm["output_ids"]) - (rm["mtp_verifications"] + rm["mtp_accepted_tokens"]) in (0, 1)
    streamed, _ = run(model, ["--max-tokens", "12", "--mtp", "--stream"], TEXT)
    assert streamed + "\n" == out


def test_qsa_budgets(model, model_dir, monkeypatch):
    # --qsa-budget: a budget above the context keeps dense attention's tokens with no
    # sparse queries; a small one selects fewer keys than dense attention would see; with
    # --mtp the output stays that of the same budget's greedy loop (Main.swift:254-276)
    monkeypatch.setenv("PLAMO_SOURCE_SHA256", model_dir[1])
    out, m = run(model, ["--max-tokens", "24"], TEXT)
    wide_out, wide = run(model, ["--max-tokens", "24", "--qsa-budget", "2048"], TEXT)
    r, rw = m["runs"][0], wide["runs"][0]
    assert wide["qsa"] is True and wide["qsa_budget"] == 2048
    # no indexer is loaded for a budget the context does not exceed (Runtime.swift:248)
    assert wide["auxiliary_weight_bytes"] == 0
    assert rw["output_ids"] == r["output_ids"] and rw["qsa_queries"] == 0
    small_out, small = run(model, ["--max-tokens", "24", "--qsa-budget", "16"], TEXT)
    rs = small["runs"][0]
    assert small["auxiliary_weight_bytes"] == 2 * 2 * (640 * 1536 + 2 * 128)
    assert rs["qsa_queries"] > 0 and rs["qsa_selected_keys"] < rs["qsa_dense_keys"]
    both_out, both = run(model, ["--max-tokens", "24", "--qsa-budget", "16", "--mtp"], TEXT)
    assert both["runs"][0]["output_ids"] == rs["output_ids"] and both_out == small_out


def test_batch4_matches_sequential_command(model):
    # BatchCLITests.swift:5-60 restated on the synthetic model: the same text through the
    # sequential segment loop and through --batch4 gives the same stdout, ids, stop reason
    # and segment count, for plain and streamed output and a short limit; the batch adds
    # KV and scratch, not another copy of the weights; --repeat 2 repeats the run exactly
    source = "\tThe meeting has been moved to next Monday.\r\n\r\n Hello.\nThank you.\nYes.\nNo.\n  "
    base = ["--segment-tokens", "64", "--to", "ja", "--max-tokens", "6"]
    for flags in (["--stream"], [], ["--stream", "--max-tokens", "3"]):
        s_out, s = run(model, base + flags, source)
        b_out, b = run(model, base + flags + ["--batch4"], source)
        sr, br = s["runs"][0], b["runs"][0]
        assert s_out == b_out and sr["output_ids"] == br["output_ids"], flags
        assert sr["stop_reason"] == br["stop_reason"] and sr["segments_total"] == br["segments_total"] > 1
        assert s["batch4"] is False and b["batch4"] is True
        assert s["gpu_weight_bytes"] == b["gpu_weight_bytes"]
        assert b["metal_allocated_bytes"] - s["metal_allocated_bytes"] < b["gpu_weight_bytes"] // 2
        assert b["peak_metal_allocated_bytes"] >= b["metal_allocated_bytes"]
    expected, _ = run(model, base, source)
    repeated, r = run(model, base + ["--batch4", "--repeat", "2"], source)
    assert repeated == expected  # the translation is printed once, the runs are counted twice
    assert len(r["runs"]) == 2 and r["runs"][0]["output_ids"] == r["runs"][1]["output_ids"]
