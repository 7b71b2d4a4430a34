"""Bit-exact decode: the GPU decode step equals the order-exact CPU restatement
(oracle/exact.py) in every logit bit, hidden bit, KV bit and token.

Config 1 in full: the 64-token prompt consumed through the decode step (Runtime.forward of
one token, Runtime.swift:321-467), then 31 greedy steps -- 95 steps, plain BF16; a shorter
run with the .p12 weights; and the sampling controls (Sampler.select over generated-only
history, Main.swift:237-244) on the device against the restated select on exact logits.
"""
import numpy as np
import pytest

import plamo_hip
from oracle import exact, sampler
from oracle.bf16 import bf_np

pytestmark = pytest.mark.gpu


def run_pair(rt, ex, prompt, decode, check_kv=True):
    nxt, ids = None, []
    for pos in range(len(prompt) + decode):
        t = prompt[pos] if pos < len(prompt) else nxt
        if pos >= len(prompt):
            ids.append(t)
        got = rt.forward([t])
        bits, hidden, want = ex.step(t, pos)
        assert np.array_equal(rt.logit_bits(), bits), pos
        assert np.array_equal(rt.hidden().view(np.uint32), hidden.view(np.uint32)), pos
        assert got == want, pos
        nxt = got
        if pos % 16 == 15:
            print(f"  bit-exact through step {pos}", flush=True)
    if check_kv:
        n = len(prompt) + decode
        for layer in range(16):
            k, v = rt.kv(layer)
            assert np.array_equal(k[:n], ex.keys[layer][:n]) and np.array_equal(v[:n], ex.values[layer][:n]), layer
    return ids


def test_config1_decode_bit_exact(model_dir, oracle_weights, golden):
    d, _ = model_dir
    rt = plamo_hip.Runtime(d, 96)
    ex = exact.ExactDecoder(oracle_weights, 96, rt.stats()["local_capacity"])
    ids = run_pair(rt, ex, golden["config1"]["prompt"], 31)
    assert len(ids) == 31
    rt.close()


def test_packed_decode_bit_exact(model_dir, oracle_weights, golden):
    d, sha = model_dir
    rt = plamo_hip.Runtime(d, 32, packed=True, source_sha256=sha)
    ex = exact.ExactDecoder(oracle_weights, 32, rt.stats()["local_capacity"])
    run_pair(rt, ex, golden["config1"]["prompt"][:6], 6)
    rt.close()


def test_sampling_controls_bit_exact(model_dir, oracle_weights, golden):
    d, _ = model_dir
    penalty, frequency, ngram = 1.1, 0.2, 4
    rt = plamo_hip.Runtime(d, 64)
    ex = exact.ExactDecoder(oracle_weights, 64, rt.stats()["local_capacity"])
    prompt = golden["config1"]["prompt"][:8]
    rt.set_sampling(penalty, frequency, 0.0, ngram)
    for pos, t in enumerate(prompt[:-1]):
        rt.forward([t])
        ex.step(t, pos)
    generated = []
    nxt = rt.forward([prompt[-1]])
    bits, _, _ = ex.step(prompt[-1], len(prompt) - 1)
    assert nxt == sampler.select(bf_np(bits).copy(), generated, penalty, ngram, frequency)
    pos = len(prompt)
    for _ in range(20):
        if nxt in (1, 16):
            break
        generated.append(nxt)
        rt.observe(nxt)
        t = nxt
        nxt = rt.forward([t])
        bits, _, _ = ex.step(t, pos)
        pos += 1
        assert np.array_equal(rt.logit_bits(), bits)
        assert nxt == sampler.select(bf_np(bits).copy(), generated, penalty, ngram, frequency)
    rt.close()


@pytest.mark.parametrize("prompt_len", [128, 190, 320])
def test_decode_merges_in_the_o_projection_bit_exact(model_dir, oracle_weights, prompt_len):
    # rows of 2..6 attention partitions (129..384 keys) are merged by the o projection's
    # prologue instead of the attention kernel: the twin (which merges in partition order,
    # oracle/exact.py) must still match bit for bit.  The GPU's KV after a plain prefill is
    # handed to the twin, as in the long-context test; 3-6 partitions are crossed on the way.
    d, _ = model_dir
    rt = plamo_hip.Runtime(d, prompt_len + 80)
    prompt = np.random.default_rng(prompt_len).integers(1024, 107520, prompt_len).tolist()
    t = rt.prefill(prompt)
    ex = exact.ExactDecoder(oracle_weights, prompt_len + 80, rt.stats()["local_capacity"])
    for layer in range(16):
        k, v = rt.kv(layer)
        ex.keys[layer][:] = k
        ex.values[layer][:] = v
    for pos in range(prompt_len, prompt_len + 6):
        got = rt.forward([t])
        bits, hidden, want = ex.step(t, pos)
        assert np.array_equal(rt.logit_bits(), bits), pos
        assert np.array_equal(rt.hidden().view(np.uint32), hidden.view(np.uint32)), pos
        assert got == want, pos
        t = got
    for layer in range(16):
        k, v = rt.kv(layer)
        n = prompt_len + 6
        assert np.array_equal(k[:n], ex.keys[layer][:n]) and np.array_equal(v[:n], ex.values[layer][:n]), layer
    print(f"  positions {prompt_len}..{prompt_len + 5}: bit-exact", flush=True)
    rt.close()
