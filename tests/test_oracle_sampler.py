"""Sampler, argmax and decodeBatch restatements pinned by the reference's KATs."""
import itertools

import numpy as np
import pytest

from oracle import sampler


# ---- Sampler.select (SamplerTests.swift:5-32)
def test_greedy_picks_first_maximum():
    assert sampler.select(np.array([1, 2, 2, 0], np.float32), [], 1, 0) == 1


def test_repetition_penalty_moves_choice():
    assert sampler.select(np.array([1, 5, 4], np.float32), [1], 2, 0) == 2
    assert sampler.select(np.array([-1, -5, -4], np.float32), [1], 2, 0) == 0


def test_frequency_penalty_compounds_with_count():
    assert sampler.select(np.array([0, 5, 4], np.float32), [1], 1, 0, frequency=0.5) == 1
    assert sampler.select(np.array([0, 5, 4], np.float32), [1, 1, 1], 1, 0, frequency=0.5) == 2


def test_forbidden_ngrams_block_the_completion():
    assert sampler.forbidden([0, 2, 3, 5, 2, 3], 3) == {5}
    assert sampler.select(np.array([0, 0, 0, 0, 0, 9], np.float32), [0, 2, 3, 5, 2, 3], 1, 3) == 0


def test_forbidden_brute_force_small_histories():
    # independent definition over completion indices j: h[j] is banned when the n-1 tokens
    # before it equal the trailing n-1 tokens of the history (j < len, so the trailing
    # n-gram itself never bans anything)
    for n in (2, 3, 4):
        for hist in itertools.product(range(3), repeat=6):
            h = list(hist)
            tail = h[len(h) - (n - 1):]
            want = {h[j] for j in range(n - 1, len(h)) if h[j - (n - 1):j] == tail}
            assert sampler.forbidden(h, n) == want


def test_select_nan_and_all_inf():
    assert sampler.select(np.array([np.nan, np.nan], np.float32), [], 1, 0) == 0
    assert sampler.select(np.array([-np.inf, -np.inf], np.float32), [], 1, 0) == 0


# ---- argmax (ArgmaxTests.swift:13-59)
def argmax_patterns():
    for count in [1, 31, 32, 33, 255, 256, 257, 1023, 1024, 1025]:
        for pattern in range(5):
            v = (np.arange(count) * 17 % 4093 - 2046).astype(np.float32) / 32
            if pattern == 1:
                v[:] = -np.inf
            elif pattern == 2:
                v[:] = np.nan
            elif pattern == 3:
                v = np.where(np.arange(count) % 2 == 0, np.float32(-0.0), np.float32(0.0)).astype(np.float32)
            elif pattern == 4:
                v[0] = np.nan
                if count > 1:
                    v[count - 1] = np.inf
                if count > 257:
                    v[257] = np.inf
            yield count, pattern, v


def test_argmax_matches_sequential_definition():
    for count, pattern, v in argmax_patterns():
        assert sampler.argmax_gpu(v) == sampler.argmax_sequential(v), (count, pattern)
    assert sampler.argmax_gpu(np.full(5, np.nan, np.float32)) == 0xFFFFFFFF
    assert sampler.argmax_gpu(np.full(5, -np.inf, np.float32)) == 0


# ---- decodeBatch (OrderedTests.swift:25-66)
def bytes_ids(text):
    return [b + 384 if b < 128 else b for b in text.encode()]


def simulate(texts, limits, stop_on_truncation=True, run=sampler.decode_batch):
    source = [bytes_ids(t) for t in texts]
    cursor = [0] * len(texts)
    calls = []

    def nxt():
        return [source[i][cursor[i]] if cursor[i] < len(source[i]) else (1 if i % 2 == 0 else 16)
                for i in range(len(source))]

    def step(tokens):
        calls.append(list(tokens))
        for lane, t in enumerate(tokens):
            if t is not None:
                assert t == source[lane][cursor[lane]]
                cursor[lane] += 1
        return nxt()

    return run(nxt(), limits, step, stop_on_truncation=stop_on_truncation), calls


def test_decode_batch_future_eos():
    out, _ = simulate(["AAA", "B", "あ", ""], [20, 20, 20, 20])
    assert [r for _, r in out] == ["stop"] * 4
    assert out[2][0] == list("あ".encode())


def test_decode_batch_later_truncation():
    out, calls = simulate(["AAA", "BBBB", "C", "DDDD"], [20, 2, 20, 20])
    assert [r for _, r in out] == ["stop", "length"]
    assert [ids for ids, _ in out] == [bytes_ids("AAA"), bytes_ids("BB")]
    assert calls[0] == [449, 450, 451, 452]
    assert all(c[1] is None and c[2] is None and c[3] is None for c in calls[1:])
    early, _ = simulate(["AAAA", "BBBB", "CCCC", "D"], [2, 20, 1, 20])
    assert [r for _, r in early] == ["length"]
    zero, zcalls = simulate(["A", "B"], [0, 20])
    assert zcalls == []


def test_decode_batch_finish_order_independent_mode():
    calls, finished, pending = [], [], [[1, 16, 100, 201], [1, 16, 100, 202]]

    def step(t):
        calls.append(list(t))
        return pending.pop(0)

    out = sampler.decode_batch([1, 16, 100, 200], [9, 9, 1, 3], step, finish=lambda lane, _: finished.append(lane))
    assert [ids for ids, _ in out] == [[], [], [100], [200, 201, 202]]
    assert [r for _, r in out] == ["stop", "stop", "length", "length"]
    assert calls == [[None, None, None, 200], [None, None, None, 201]]
    assert finished == [0, 1, 2, 3]


def test_decode_batch_rejects_invalid():
    with pytest.raises(ValueError):
        sampler.decode_batch([107520], [1], lambda t: t)
    with pytest.raises(ValueError):
        sampler.decode_batch([5], [8192], lambda t: t)
