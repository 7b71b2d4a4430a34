"""Long context (config 5) and wrapped rings (config 4) on the GPU.

Config 5: a 30,720-token prompt prefilled from the .p12 weights (15 MFMA chunks of 2048),
then decode with the sampling controls at positions 30,720 and up.  The GPU KV cache after
the prefill is handed to the order-exact CPU decoder (oracle/exact.py), and every following
decode step must match it bit for bit: logits, final hidden state, the new KV rows and the
controlled selection (Sampler.select over the generated history, Main.swift:237-244).  This
covers the ring wrap of the 14 local layers, global attention over ~30K keys in 480
partitions and the split-K merge at that size.  The device loop then runs the whole config
(2,048 generated tokens) to the 32,768 cap, and its last eight positions are checked the same
way.  The MFMA prefill is held bit-exact by tests/test_gpu_prefill_exact.py.

Config 4 itself: four segments with 512/384/256/128-token prompts, each greedy-decoding up
to 2048 tokens (stop ids 1 and 16) at context 2,560 in the batch device loop; every lane's
ids equal scalar generation of its prompt and, at the end, its logits, hidden row and every
layer's KV equal the scalar runtime's bit for bit (Batch.swift:109-180 keeps lanes
independent).  A shorter variant steps the batch by hand until the longest lane attends over
a 2048-key window that no longer starts at position 0.  (Lane rings wrap in
tests/test_gpu_batch.py's "wrap" case: this build's local ring holds 2048 + one 2048-token
prefill chunk, more than configs[3]'s context.)
"""
import time

import numpy as np
import pytest

import plamo_hip
from oracle import exact, sampler
from oracle.bf16 import bf_np

pytestmark = pytest.mark.gpu

PENALTY, FREQUENCY, NGRAM = 1.1, 0.2, 4


@pytest.fixture(scope="module")
def long_runtime(model_dir):
    d, sha = model_dir
    rt = plamo_hip.Runtime(d, 32768, packed=True, source_sha256=sha)
    yield rt
    rt.close()


def long_prompt():
    return np.random.default_rng(5).integers(1024, 107520, 30720).tolist()


def test_long_context_decode_bit_exact(long_runtime, oracle_weights):
    rt = long_runtime
    rt.reset()
    rt.set_sampling(PENALTY, FREQUENCY, 0.0, NGRAM)
    try:
        t0 = time.time()
        nxt = rt.prefill(long_prompt())
        print(f"  prefill 30720 tokens (.p12): {time.time() - t0:.2f} s", flush=True)
        ex = exact.ExactDecoder(oracle_weights, 32768, rt.stats()["local_capacity"])
        for layer in range(16):
            k, v = rt.kv(layer)
            ex.keys[layer][:] = k
            ex.values[layer][:] = v
        generated, pos, t = [], 30720, nxt
        for step in range(6):
            generated.append(t)
            rt.observe(t)
            got = rt.forward([t])
            bits, hidden, _ = ex.step(t, pos)
            assert np.array_equal(rt.logit_bits(), bits), step
            assert np.array_equal(rt.hidden().view(np.uint32), hidden.view(np.uint32)), step
            assert got == sampler.select(bf_np(bits).copy(), generated, PENALTY, NGRAM, FREQUENCY), step
            print(f"  position {pos}: bit-exact, token {got}", flush=True)
            t, pos = got, pos + 1
        for layer in range(16):
            k, v = rt.kv(layer)
            cap = k.shape[0]
            slots = [p % cap for p in range(30720, pos)]
            assert np.array_equal(k[slots], ex.keys[layer][slots]), layer
            assert np.array_equal(v[slots], ex.values[layer][slots]), layer
    finally:
        rt.set_sampling()


def test_decode_crosses_the_first_window_bit_exact(model_dir, oracle_weights):
    # Inside the first window (positions < 2048) local-layer attention reads keys rotated at
    # their own position, cached when each key was written (by the prefill and by decode);
    # from 2048 on it rotates the unrotated keys by position - (pos - 2047).  Decode across
    # the switch, from a GPU prefill handed to the CPU decoder, bit for bit.
    d, _ = model_dir
    rt = plamo_hip.Runtime(d, 2112)
    try:
        nxt = rt.prefill(np.random.default_rng(9).integers(1024, 107520, 2030).tolist())
        ex = exact.ExactDecoder(oracle_weights, 2112, rt.stats()["local_capacity"])
        for layer in range(16):
            k, v = rt.kv(layer)
            ex.keys[layer][:] = k
            ex.values[layer][:] = v
        t, pos = nxt, 2030
        for step in range(30):
            got = rt.forward([t])
            bits, hidden, want = ex.step(t, pos)
            assert np.array_equal(rt.logit_bits(), bits), pos
            assert np.array_equal(rt.hidden().view(np.uint32), hidden.view(np.uint32)), pos
            assert got == want, pos
            if pos in (2047, 2048, 2059):
                print(f"  position {pos}: bit-exact", flush=True)
            t, pos = got, pos + 1
        for layer in range(16):
            k, v = rt.kv(layer)
            slots = [p % k.shape[0] for p in range(2030, pos)]
            assert np.array_equal(k[slots], ex.keys[layer][slots]), layer
    finally:
        rt.close()


def test_long_context_runs_to_the_cap_bit_exact(long_runtime, oracle_weights):
    # Config 5 end to end: the device loop generates from the 30,720-token prompt to within
    # a few positions of the 32,768 cap (sampling controls over the generated history), the
    # CPU decoder takes over the GPU's KV there, and the last forwards up to position 32,767
    # match it bit for bit; one more forward is refused (Runtime.swift:328-330).
    rt = long_runtime
    tail = 7
    rt.set_sampling(PENALTY, FREQUENCY, 0.0, NGRAM)
    try:
        t0 = time.time()
        ids, reason = rt.generate(long_prompt(), 2048 - tail)
        print(f"  device loop: {len(ids)} tokens in {time.time() - t0:.2f} s, reason {reason}", flush=True)
        assert reason is None and len(ids) == 2048 - tail
        pos = rt.position
        assert pos == 30720 + len(ids) - 1, pos
        ex = exact.ExactDecoder(oracle_weights, 32768, rt.stats()["local_capacity"])
        for layer in range(16):
            k, v = rt.kv(layer)
            ex.keys[layer][:] = k
            ex.values[layer][:] = v
        generated, t, start = list(ids), ids[-1], pos
        while pos < 32768:
            got = rt.forward([t])
            bits, hidden, _ = ex.step(t, pos)
            assert np.array_equal(rt.logit_bits(), bits), pos
            assert np.array_equal(rt.hidden().view(np.uint32), hidden.view(np.uint32)), pos
            assert got == sampler.select(bf_np(bits).copy(), generated, PENALTY, NGRAM, FREQUENCY), pos
            print(f"  position {pos}: bit-exact, token {got}", flush=True)
            t, pos = got, pos + 1
            generated.append(t)
            rt.observe(t)
        assert rt.position == 32768
        # MaximumTests.swift:69-72: past the cap a forward is refused, the position and the
        # logits stay
        last = rt.logit_bits().copy()
        with pytest.raises(plamo_hip.PlamoError, match="context exhausted"):
            rt.forward([t])
        assert rt.position == 32768 and np.array_equal(rt.logit_bits(), last)
        for layer in range(16):
            k, v = rt.kv(layer)
            slots = [p % k.shape[0] for p in range(start, 32768)]
            assert np.array_equal(k[slots], ex.keys[layer][slots]), layer
            assert np.array_equal(v[slots], ex.values[layer][slots]), layer
    finally:
        rt.set_sampling()


def test_long_context_device_loop_matches_host_loop(long_runtime):
    rt = long_runtime
    rt.set_sampling(PENALTY, FREQUENCY, 0.0, NGRAM)
    try:
        rt.reset()
        ids, _ = rt.generate(long_prompt(), 12)
        rt.reset()
        nxt = rt.prefill(long_prompt())
        host = []
        for i in range(12):
            if nxt in (1, 16):
                break
            host.append(nxt)
            rt.observe(nxt)
            if i + 1 < 12:
                nxt = rt.forward([nxt])
    finally:
        rt.set_sampling()
    assert ids == host


def test_batch_segments_cross_the_window(model_dir):
    d, _ = model_dir
    lengths = [512, 384, 256, 128]
    steps = 2048 + 40 - 512
    rng = np.random.default_rng(11)
    prompts = [rng.integers(1024, 107520, n).tolist() for n in lengths]
    rt = plamo_hip.Runtime(d, 2200)
    b = plamo_hip.Batch(rt)
    try:
        tokens = b.prefill(prompts)
        for _ in range(steps):
            tokens = b.step(tokens)
        print(f"  batch decoded {steps} steps, positions {b.positions()}", flush=True)
        for lane, p in enumerate(prompts):
            rt.reset()
            nxt = rt.prefill(p)
            for _ in range(steps):
                nxt = rt.forward([nxt])
            assert tokens[lane] == nxt, lane
            assert np.array_equal(b.logit_bits(lane), rt.logit_bits()), lane
            assert np.array_equal(b.hidden(lane).view(np.uint32), rt.hidden().view(np.uint32)), lane
            n = len(p) + steps
            for layer in (0, 7):
                kb, vb = b.kv(lane, layer)
                ks, vs = rt.kv(layer)
                assert np.array_equal(kb[:n], ks[:n]) and np.array_equal(vb[:n], vs[:n]), (lane, layer)
            print(f"  lane {lane} (prompt {len(p)}): batch == scalar", flush=True)
    finally:
        b.close()
        rt.close()


def test_config4_batch_runs_to_its_horizon(model_dir):
    d, _ = model_dir
    lengths, limit, context = (512, 384, 256, 128), 2048, 2560
    # the bench's configs[3] prompts
    prompts = [np.random.default_rng(20 + i).integers(1024, 107520, n).tolist() for i, n in enumerate(lengths)]
    rt = plamo_hip.Runtime(d, context)
    b = plamo_hip.Batch(rt)
    try:
        t0 = time.time()
        outs = b.generate(prompts, [limit] * 4)
        print(f"  batch device loop: {[len(ids) for ids, _ in outs]} tokens, reasons "
              f"{[r for _, r in outs]} in {time.time() - t0:.2f} s", flush=True)
        lanes = [(b.logit_bits(lane).copy(), b.hidden(lane).copy(), [b.kv(lane, layer) for layer in range(16)])
                 for lane in range(4)]
        positions = b.positions()
        for lane, p in enumerate(prompts):
            rt.reset()
            ids, reason = rt.generate(p, limit)
            assert ids == outs[lane][0], lane
            assert outs[lane][1] == ("stop" if reason == "stop" else "length"), lane
            assert positions[lane] == rt.position, lane
            logits, hidden, kv = lanes[lane]
            assert np.array_equal(logits, rt.logit_bits()), lane
            assert np.array_equal(hidden.view(np.uint32), rt.hidden().view(np.uint32)), lane
            n = rt.position
            for layer in range(16):
                ks, vs = rt.kv(layer)
                kb, vb = kv[layer]
                assert np.array_equal(kb[:n], ks[:n]) and np.array_equal(vb[:n], vs[:n]), (lane, layer)
            print(f"  lane {lane} (prompt {len(p)}): {len(ids)} tokens ({outs[lane][1]}), position {n}: "
                  "batch == scalar", flush=True)
    finally:
        b.close()
        rt.close()
