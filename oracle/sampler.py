"""Token selection and the lane scheduler (test infrastructure only).

* ``argmax_gpu``     -- ``argmax`` (Kernels.metal:704-729): first index of the maximum, NaN
  never wins, an all-NaN row gives 0xffffffff.  Pinned by the pattern set of
  ``Tests/PlamoTests/ArgmaxTests.swift:13-59`` (whose in-test expectation loop is the
  sequential definition restated in ``argmax_sequential``).
* ``select``         -- ``Sampler.select`` (Sampler.swift:9-32): FP32 repetition penalty
  (divide if positive, multiply otherwise), presence, frequency x count, n-gram ban to -inf,
  then the first strict maximum with default 0.  Pinned by the five KATs of
  ``Tests/PlamoTests/SamplerTests.swift:5-32``.
* ``forbidden``      -- ``Sampler.forbidden`` (Sampler.swift:54-70).  Pinned by
  ``SamplerTests.swift:26-29`` and brute force over all short histories in tests.
* ``decode_batch``   -- ``decodeBatch`` (BatchDecode.swift:8-37).  Pinned by
  ``Tests/PlamoTests/OrderedTests.swift:25-66`` (id sequences, reasons, step calls and
  finish order).
"""
import numpy as np

VOCAB = 107520
STOP = (1, 16)


def argmax_gpu(values):
    v = np.asarray(values, dtype=np.float32)
    ok = ~np.isnan(v)
    if not ok.any():
        return 0xFFFFFFFF
    m = v[ok].max()
    return int(np.flatnonzero(ok & (v == m))[0])


def argmax_sequential(values):
    """The expectation loop of ArgmaxTests.swift:31-37."""
    best, index = -np.inf, 0xFFFFFFFF
    for i, value in enumerate(np.asarray(values, dtype=np.float32).tolist()):
        if value > best or (value == best and i < index):
            best, index = value, i
    return index


def forbidden(history, n):
    if n <= 1 or len(history) < n:
        return set()
    span = n - 1
    last = len(history) - span
    tail = list(history[last:])
    return {history[s + span] for s in range(last) if list(history[s:s + span]) == tail}


def select(logits, history, penalty, no_repeat_ngram, frequency=0.0, presence=0.0):
    """Sampler.select on an FP32 array (modified in place); returns the chosen index."""
    logits = np.asarray(logits, dtype=np.float32)
    penalty, frequency, presence = np.float32(penalty), np.float32(frequency), np.float32(presence)
    if penalty != 1 or presence != 0 or frequency != 0:
        counts = {}
        for i in history:
            if 0 <= i < len(logits):
                counts[i] = counts.get(i, 0) + 1
        for i, c in counts.items():
            if penalty != 1:
                logits[i] = logits[i] / penalty if logits[i] > 0 else logits[i] * penalty
            if presence != 0:
                logits[i] = logits[i] - presence
            if frequency != 0:
                logits[i] = logits[i] - np.float32(frequency * np.float32(c))
    if no_repeat_ngram > 1:
        for i in forbidden(list(history), no_repeat_ngram):
            if 0 <= i < len(logits):
                logits[i] = -np.inf
    best, index = -np.inf, 0
    for i, value in enumerate(logits.tolist()):
        if value > best:
            best, index = value, i
    return index


def decode_batch(initial, limits, step, emit=None, finish=None, stop_on_truncation=False):
    """decodeBatch (BatchDecode.swift:8-37) -> list of (ids, reason)."""
    count = len(initial)
    if not (1 <= count <= 4) or any(not (0 <= t < VOCAB) for t in initial) or \
            len(limits) != count or any(not (0 <= l <= 8191) for l in limits):
        raise ValueError("Invalid quad decode inputs")
    nxt, outputs, reasons = list(initial), [[] for _ in range(count)], [None] * count
    last = count - 1
    while any(r is None for r in reasons[:last + 1]):
        tokens = [None] * count
        for lane in range(count):
            if lane > last:
                break
            if reasons[lane] is not None:
                continue
            if len(outputs[lane]) == limits[lane]:
                reasons[lane] = "length"
            elif nxt[lane] in STOP:
                reasons[lane] = "stop"
            else:
                outputs[lane].append(nxt[lane])
                if emit:
                    emit(lane, nxt[lane])
                if len(outputs[lane]) == limits[lane]:
                    reasons[lane] = "length"
                else:
                    tokens[lane] = nxt[lane]
            if reasons[lane] is not None:
                if stop_on_truncation and reasons[lane] == "length":
                    last = min(last, lane)
                if finish:
                    finish(lane, (list(outputs[lane]), reasons[lane]))
        if all(t is None for t in tokens):
            break
        nxt = step(tokens)
        if len(nxt) != count or any(not (0 <= t < VOCAB) for t in nxt):
            raise ValueError("Invalid quad predictions")
    return [(outputs[i], reasons[i]) for i in range(last + 1)]
