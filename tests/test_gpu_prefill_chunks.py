"""Prefill over several chunks (Runtime.prefill, Runtime.swift:469-483) bit-exact against the
order-exact CPU restatement (oracle/exact_prefill.py).

The runtime runs a prompt in 2048-token chunks.  From position 2048 on, local-layer RoPE
coordinates are relative to a base above 0 (Runtime.swift:389-399), the flash kernel's
queries see keys written by an earlier chunk, and past position 4096 a chunk's keys wrap the
4,096-slot local rings while its queries attend over the wrapped window.

* two chunks (2,344 tokens): the twin runs layer 0 in full and layer 1 up to its KV write,
  chunk by chunk, and every key and value word of both layers equals the GPU's;
* three chunks (4,200 tokens at context 4,400, rings wrapping in the third): all 16 layers'
  cached rows, the last token's logits and hidden row and the next token hash to the
  digests of the full twin (tests/golden/make_chunked_digest.py), plain and .p12; greedy
  decode then continues bit-exactly from that state against the decode twin.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import plamo_hip
from oracle import exact, exact_prefill as xp

pytestmark = pytest.mark.gpu

DIGEST = os.path.join(os.path.dirname(__file__), "golden", "chunked_prefill_digest.json")


def _digest(a, dtype):
    return hashlib.sha256(np.ascontiguousarray(a, dtype=dtype).tobytes()).hexdigest()


def test_two_chunk_prefill_first_layers_bit_exact(model_dir, oracle_weights):
    prompt = np.random.default_rng(21).integers(1024, 107520, 2048 + 296).tolist()
    n = len(prompt)
    d, _ = model_dir
    rt = plamo_hip.Runtime(d, 2400)
    try:
        rt.prefill(prompt)
        kv = [rt.kv(layer) for layer in (0, 1)]
        cap = rt.stats()["local_capacity"]
    finally:
        rt.close()
    print(f"  GPU prefill of {n} tokens in two chunks done; running the twin (layers 0-1)", flush=True)
    ex = exact.ExactDecoder(oracle_weights, 2400, cap)
    xp.ExactPrefill(ex).prefill(prompt, kv_layers=2)
    for layer, (k, v) in zip((0, 1), kv):
        bad_k = int(np.sum(k[:n] != ex.keys[layer][:n]))
        bad_v = int(np.sum(v[:n] != ex.values[layer][:n]))
        print(f"  two chunks, layer {layer}: {bad_k} key / {bad_v} value words differ", flush=True)
        assert bad_k == 0 and bad_v == 0, layer


@pytest.fixture(scope="module")
def chunked_case(model_dir):
    with open(DIGEST) as f:
        want = json.load(f)
    d, sha = model_dir
    assert want["model_sha256"] == sha
    prompt = np.random.default_rng(want["prompt_seed"]).integers(1024, 107520, want["prompt_tokens"]).tolist()
    return want, prompt


@pytest.mark.parametrize("packed", [False, True])
def test_chunked_prefill_matches_twin_digests(model_dir, oracle_weights, chunked_case, packed):
    want, prompt = chunked_case
    n = len(prompt)
    d, sha = model_dir
    rt = plamo_hip.Runtime(d, want["context"], packed=packed, source_sha256=sha)
    try:
        assert rt.stats()["local_capacity"] == want["local_capacity"]
        nxt = rt.prefill(prompt)
        bad = []
        kv = [rt.kv(layer) for layer in range(16)]
        for layer, (k, v) in enumerate(kv):
            rows = min(n, k.shape[0])
            for name, a in (("keys", k[:rows]), ("values", v[:rows])):
                if _digest(a, np.uint16) != want["layers"][layer][name]:
                    bad.append(f"layer {layer} {name}")
        if _digest(rt.logit_bits(), np.uint16) != want["logits"]:
            bad.append("logits")
        if _digest(rt.hidden().view(np.uint32), np.uint32) != want["hidden"]:
            bad.append("hidden")
        print(f"  {n}-token prefill in 3 chunks (packed={packed}): next {nxt} (twin {want['next']}), "
              f"differing: {bad or 'none'}", flush=True)
        assert not bad, bad
        assert nxt == want["next"]
        if packed:
            return
        # the GPU state now equals the twin's in every cached word: decode continues from it
        # bit for bit against the decode twin (wrapped rings, window starting above 0)
        ex = exact.ExactDecoder(oracle_weights, want["context"], want["local_capacity"])
        for layer, (k, v) in enumerate(kv):
            ex.keys[layer][:] = k
            ex.values[layer][:] = v
        t, pos = nxt, n
        for _ in range(4):
            got = rt.forward([t])
            bits, hidden, nxt2 = ex.step(t, pos)
            assert np.array_equal(rt.logit_bits(), bits), pos
            assert np.array_equal(rt.hidden().view(np.uint32), hidden.view(np.uint32)), pos
            assert got == nxt2, pos
            print(f"  position {pos}: bit-exact, token {got}", flush=True)
            t, pos = got, pos + 1
    finally:
        rt.close()
