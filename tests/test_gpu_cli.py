"""The plamo command (plamo_hip.cli) end to end on the GPU with the synthetic model.

Checks the stderr metrics schema (Main.swift:331-347 top-level keys, 265-273 run keys), that
the command's tokens equal the runtime's own greedy loop, --stream text equal to the plain
text, --dump-logits, and the segment pipeline's stop rule (SegmentTests.swift:97-107: a
truncated segment stops the pipeline; the synthetic model's random weights rarely stop, so
only the first segment is translated)."""
import io
import json
import os

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
    if m1["runs"][0]["stop_reason"] == "length":
        assert chunked == first and r["stop_reason"] == "length" and r["segments_completed"] == 0
        assert r["output_ids"] == m1["runs"][0]["output_ids"]
    _, b = run(model, ["--to", "en", "--max-tokens", "4", "--segment-tokens", "64", "--batch4"], UNBROKEN)
    rb = b["runs"][0]
    assert {"prefilled_input_tokens", "discarded_output_tokens", "segments", "segments_total"} <= set(rb)
    assert rb["segments"][0]["output_ids"] == m1["runs"][0]["output_ids"]
    tok.close()
