"""batch4: every lane's state is bit-equal to scalar decode of the same prompt
(BatchMapTests.swift:6-73), for every subset of active lanes."""
import numpy as np
import pytest

import plamo_hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def engines(model_dir):
    d, sha = model_dir
    rt = plamo_hip.Runtime(d, 160)
    b = plamo_hip.Batch(rt)
    yield rt, b
    b.close()
    rt.close()


def prompts_for(lengths):
    return [[1] + [1000 + k * 17 for k in range(1, n)] for n in lengths]


def scalar_state(rt, prompt, steps):
    rt.reset()
    nxt = rt.prefill(prompt)
    for _ in range(steps):
        nxt = rt.forward([nxt])
    kv = [rt.kv(l) for l in range(16)]
    return nxt, rt.logit_bits().copy(), rt.hidden().copy(), kv


@pytest.mark.parametrize("lengths", [[63, 3, 7, 5], [3, 63], [1, 4, 2], [2]])
def test_batch_step_equals_scalar(engines, lengths):
    rt, b = engines
    prompts = prompts_for(lengths)
    steps = 2
    expected = [scalar_state(rt, p, steps) for p in prompts]
    tokens = b.prefill(prompts)
    for _ in range(steps):
        tokens = b.step(tokens)
    for lane, p in enumerate(prompts):
        nxt, logits, hidden, kv = expected[lane]
        assert tokens[lane] == nxt
        assert np.array_equal(b.logit_bits(lane), logits)
        assert np.array_equal(b.hidden(lane).view(np.uint32), hidden.view(np.uint32))
        n = len(p) + steps
        for layer in range(16):
            k, v = b.kv(lane, layer)
            assert np.array_equal(k[:n], kv[layer][0][:n]) and np.array_equal(v[:n], kv[layer][1][:n]), layer


def test_lane_subsets(engines):
    # masks 1..15 of active lanes: inactive lanes keep their state untouched
    rt, b = engines
    prompts = prompts_for([9, 5, 12, 3])
    for mask in range(1, 16):
        first = b.prefill(prompts)
        tokens = [first[i] if mask >> i & 1 else None for i in range(4)]
        out = b.step(tokens)
        for lane in range(4):
            if mask >> lane & 1:
                nxt, logits, _, _ = scalar_state(rt, prompts[lane], 1)
                assert out[lane] == nxt, (mask, lane)
            else:
                assert out[lane] == first[lane]
        assert b.positions() == [len(p) + (mask >> i & 1) for i, p in enumerate(prompts)]


def test_generate_matches_sequential(engines):
    rt, b = engines
    prompts = prompts_for([20, 14, 9, 30])
    limits = [12, 5, 12, 8]
    got = b.generate(prompts, limits)
    for lane, (ids, reason) in enumerate(got):
        rt.reset()
        want, r = rt.generate(prompts[lane], limits[lane])
        assert ids == want
        assert reason == ("stop" if r == "stop" else "length")


@pytest.mark.parametrize("limits,override,trunc", [
    ([12, 5, 0, 8], {}, False),            # a zero limit ends its lane before any step
    ([6, 6, 6, 6], {1: 16, 3: 1}, False),  # stop tokens end lanes 1 and 3 at once
    ([9, 3, 9, 9], {}, True),              # lane 1 truncates: lanes 2 and 3 are dropped
    ([4, 7, 2], {0: 1}, True),             # stop (not truncation) keeps the later lanes
])
def test_device_loop_matches_host_loop(engines, limits, override, trunc):
    # the device lane pass and token feedback against decodeBatch driving Batch.step
    rt, b = engines
    prompts = prompts_for([20, 14, 9, 30][:len(limits)])
    first = b.prefill(prompts)
    initial = [override.get(i, t) for i, t in enumerate(first)]
    want = plamo_hip.decode_batch(initial, limits, b.step, stop_on_truncation=trunc)
    want_pos = b.positions()
    want_logits = [b.logit_bits(i).copy() for i in range(len(prompts))]
    want_hidden = [b.hidden(i).copy() for i in range(len(prompts))]
    assert b.prefill(prompts) == first
    got = b.decode(initial, limits, stop_on_truncation=trunc)
    assert got == want
    assert b.positions() == want_pos
    for i in range(len(prompts)):
        assert np.array_equal(b.logit_bits(i), want_logits[i]), i
        assert np.array_equal(b.hidden(i).view(np.uint32), want_hidden[i].view(np.uint32)), i


def test_batch_validation(engines, model_dir):
    rt, b = engines
    with pytest.raises(plamo_hip.PlamoError, match="Expected one to four valid prompts"):
        b.prefill([])
    b.reset()
    with pytest.raises(plamo_hip.PlamoError, match="Invalid quad step"):
        b.step([5])
    big = plamo_hip.Runtime(model_dir[0], 8192)
    try:
        with pytest.raises(plamo_hip.PlamoError, match="below 8192"):
            plamo_hip.Batch(big)
    finally:
        big.close()


def _tails(b, lengths):
    """Every lane's KV rows past its prompt (all rows of lanes without a prompt)."""
    out = []
    for lane in range(4):
        for layer in range(16):
            k, v = b.kv(lane, layer)
            used = min(lengths[lane], len(k)) if lane < len(lengths) else 0
            out.append((k[used:].copy(), v[used:].copy()))
    return out


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("case", ["short", "ring", "wrap"])
def test_poisoned_unused_kv_is_never_read(model_dir, packed, case):
    """BatchMapTests.swift:6-73: the batch KV filled with NaN (BF16 0xffff); prefill leaves the
    rows past each prompt untouched, and after the steps every lane's logits, hidden row and
    written KV rows equal scalar decode of its prompt (a NaN that reached attention would
    show in all of them).  "ring" keeps the reference's second configuration (context 2100,
    a 2063-token prompt); this build's local ring holds 2100 slots there, so it does not
    wrap.  "wrap" does: at context 4400 the local rings hold 4096 slots, and lanes 0 and 2
    decode from positions 4090 and 4093 past 4096, so their newest keys go to slots 0.. of
    their own ring slice while their windows still read the slots before the wrap."""
    d, sha = model_dir
    context, steps, layouts = {
        "short": (128, 1, [[63, 3, 7, 5], [3, 63], [1, 4, 2], [2]]),
        "ring": (2100, 2, [[2063, 3], [3, 4]]),
        "wrap": (4400, 12, [[4090, 3, 4093, 1000]]),
    }[case]
    rt = plamo_hip.Runtime(d, context, packed=packed, source_sha256=sha)
    b = plamo_hip.Batch(rt)
    try:
        if case == "wrap":
            assert rt.stats()["local_capacity"] == 4096
        b.fill_kv(0xFFFF)
        for lengths in layouts:
            prompts = prompts_for(lengths)
            expected = [scalar_state(rt, p, steps) for p in prompts]
            before = _tails(b, lengths)
            tokens = b.prefill(prompts)
            after = _tails(b, lengths)
            assert all(np.array_equal(x[0], y[0]) and np.array_equal(x[1], y[1]) for x, y in zip(before, after)), \
                ("unused KV overwritten", packed, lengths)
            for _ in range(steps):
                tokens = b.step(tokens)
            for lane, p in enumerate(prompts):
                nxt, logits, hidden, kv = expected[lane]
                assert tokens[lane] == nxt, (packed, lengths, lane)
                assert np.array_equal(b.logit_bits(lane), logits), (packed, lengths, lane)
                assert np.array_equal(b.hidden(lane).view(np.uint32), hidden.view(np.uint32))
                n = len(p) + steps
                for layer in range(16):
                    k, v = b.kv(lane, layer)
                    m = min(n, len(k))
                    assert np.array_equal(k[:m], kv[layer][0][:m]) and np.array_equal(v[:m], kv[layer][1][:m]), layer
            print(f"  {case} packed={packed} prompts {lengths}: every lane equals scalar decode after {steps} steps",
                  flush=True)
    finally:
        b.close()
        rt.close()
