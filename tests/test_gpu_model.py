"""End-to-end parity of the HIP token loop against the CPU oracle (config 1 and friends).

Tolerances (north star): logits max-abs <= 2e-2 and RMSE <= 5e-3 against the oracle's FP32
head output; greedy token IDs exact; packed-weight decode bit-identical to plain BF16.
"""
import numpy as np
import pytest
import torch

import plamo_hip
from oracle import model as om
from oracle.bf16 import bf_np

pytestmark = pytest.mark.gpu

MAX_ABS, RMSE = 2e-2, 5e-3


def check_logits(gpu_bits, oracle, label):
    ref = oracle.logits_fp32.numpy().astype(np.float64)
    got = bf_np(gpu_bits).astype(np.float64)
    err = np.abs(got - ref)
    rmse = float(np.sqrt(np.mean(err ** 2)))
    assert err.max() <= MAX_ABS and rmse <= RMSE, (label, float(err.max()), rmse)
    return float(err.max()), rmse


@pytest.fixture(scope="module")
def runtimes(model_dir):
    d, sha = model_dir
    plain = plamo_hip.Runtime(d, 96)
    packed = plamo_hip.Runtime(d, 96, packed=True, source_sha256=sha)
    yield plain, packed
    plain.close()
    packed.close()


def test_config1_prefill_logits_and_greedy_ids(runtimes, oracle_weights, golden):
    g = golden["config1"]
    plain, _ = runtimes
    plain.reset()
    o = om.Oracle(oracle_weights, 96)
    nxt = plain.prefill(g["prompt"])
    o.prefill(g["prompt"])
    check_logits(plain.logit_bits(), o, "prefill")
    ids = []
    for i in range(32):
        if nxt in (1, 16):
            break
        ids.append(nxt)
        if i + 1 < 32:
            nxt = plain.forward([nxt])
            o.forward([ids[-1]])   # teacher-forced on the emitted token
            check_logits(plain.logit_bits(), o, f"step {i}")
    assert ids == g["greedy_ids"]
    assert plain.position == 64 + 31


def test_packed_decode_is_bit_identical(runtimes, golden):
    g = golden["config1"]
    plain, packed = runtimes
    for rt in runtimes:
        rt.reset()
    a, b = plain.prefill(g["prompt"]), packed.prefill(g["prompt"])
    assert a == b and np.array_equal(plain.logit_bits(), packed.logit_bits())
    for _ in range(12):
        a, b = plain.forward([a]), packed.forward([b])
        assert a == b
        assert np.array_equal(plain.logit_bits(), packed.logit_bits())
        assert np.array_equal(plain.hidden().view(np.uint32), packed.hidden().view(np.uint32))
    for layer in (0, 7):
        ka, va = plain.kv(layer)
        kb, vb = packed.kv(layer)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)


def test_device_loop_matches_host_loop(runtimes, golden):
    g = golden["config1"]
    plain, packed = runtimes
    for rt in (plain, packed):
        ids, reason = rt.generate(g["prompt"], 32)
        assert ids == g["greedy_ids"] and reason is None
        assert rt.position == 64 + 31


def test_kv_cache_matches_oracle(runtimes, oracle_weights, golden):
    g = golden["config1"]
    plain, _ = runtimes
    plain.reset()
    o = om.Oracle(oracle_weights, 96, local_capacity=plain.stats()["local_capacity"])
    nxt = plain.prefill(g["prompt"])
    o.prefill(g["prompt"])
    for _ in range(3):
        nxt2 = plain.forward([nxt])
        o.forward([nxt])
        nxt = nxt2
    n = plain.position
    for layer in range(16):
        k, v = plain.kv(layer)
        ko = o.keys[layer].numpy().astype(np.uint16)
        vo = o.values[layer].numpy().astype(np.uint16)
        for got, want in ((k, ko), (v, vo)):
            gf, wf = bf_np(got[:n]).astype(np.float64), bf_np(want[:n]).astype(np.float64)
            mismatch = np.mean(got[:n] != want[:n])
            assert mismatch < 0.02, (layer, mismatch)
            assert np.max(np.abs(gf - wf)) <= 2 ** -6 * np.maximum(1, np.abs(wf)).max(), layer


def test_failed_forward_leaves_state(runtimes, golden):
    # WorkTests.swift:23-26 / Runtime.swift:328-330: validate before mutating
    plain, _ = runtimes
    plain.reset()
    nxt = plain.prefill(golden["config1"]["prompt"][:8])
    pos, bits = plain.position, plain.logit_bits().copy()
    with pytest.raises(plamo_hip.PlamoError, match="Invalid tokens or context exhausted"):
        plain.forward([107520])
    with pytest.raises(plamo_hip.PlamoError, match="Invalid tokens or context exhausted"):
        plain.forward(list(range(1000, 1017)))
    assert plain.position == pos and np.array_equal(plain.logit_bits(), bits)
    with pytest.raises(plamo_hip.PlamoError, match="Input exceeds context"):
        plain.prefill([1000] * 200)
    assert plain.position == pos
    assert plain.forward([nxt]) >= 0


def test_single_token_prefill_equals_forward(runtimes):
    # WorkTests.swift:17-22: prefill([t]) and forward([t]) are the same step
    plain, _ = runtimes
    plain.reset()
    a = plain.prefill([600])
    la = plain.logit_bits().copy()
    plain.reset()
    b = plain.forward([600])
    assert a == b and np.array_equal(la, plain.logit_bits())


def test_chunked_forward_matches_oracle(runtimes, oracle_weights, golden):
    # forward of 2..16 tokens runs the MFMA prefill path (Runtime.swift:372-374)
    plain, _ = runtimes
    p = golden["config1"]["prompt"]
    plain.reset()
    o = om.Oracle(oracle_weights, 96)
    for chunk in (p[:5], p[5:21], p[21:22], p[22:30]):
        plain.forward(chunk)
        o.forward(chunk)
        check_logits(plain.logit_bits(), o, f"chunk {len(chunk)}")


def test_sampling_controls_match_oracle(runtimes, golden):
    gs = golden["config1_sampling"]
    plain, packed = runtimes
    for rt in (plain, packed):
        rt.set_sampling(gs["penalty"], gs["frequency"], 0.0, gs["ngram"])
        try:
            ids, reason = rt.generate(golden["config1"]["prompt"], gs["max_tokens"])
        finally:
            rt.set_sampling()
        assert ids == gs["ids"]
        # the host-driven loop (Main.swift:278-287) gives the same ids
        rt.set_sampling(gs["penalty"], gs["frequency"], 0.0, gs["ngram"])
        try:
            rt.reset()
            nxt = rt.prefill(golden["config1"]["prompt"])
            host = []
            for i in range(gs["max_tokens"]):
                if nxt in (1, 16):
                    break
                host.append(nxt)
                rt.observe(nxt)
                if i + 1 < gs["max_tokens"]:
                    nxt = rt.forward([nxt])
        finally:
            rt.set_sampling()
        assert host == gs["ids"]
