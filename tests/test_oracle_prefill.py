"""Pins of the order-exact prefill restatement (oracle/exact_prefill.py, oracle/csrc) on the CPU."""
import os

import numpy as np
import pytest
import torch

from oracle import exact, exact_prefill as xp, rope
from oracle.bf16 import bf_np, bits_np, roundbf_np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FIXTURE = os.path.join(ROOT, "tests", "golden", "mfma_accumulate.npz")
F = np.float32


@pytest.fixture(scope="module", autouse=True)
def _lib():
    if exact._c_lib() is None:
        pytest.skip("oracle C restatement not built (make -C oracle)")


def test_model_reproduces_device_accumulators():
    # the device is the authority for MFMA rounding: every recorded accumulator, bit for bit
    from golden import make_mfma_fixture as mk
    got_all = np.load(FIXTURE)
    for name, (w, x) in mk.cases().items():
        want = got_all[name]
        got = xp.mfma_gemm(w, x)
        assert got.shape == want.shape, name
        bad = int(np.sum(got.view(np.uint32) != want.view(np.uint32)))
        assert bad == 0, (name, bad, want.size)


def _rand_bits(rng, shape, scale=1.0):
    return bits_np((rng.standard_normal(shape) * scale).astype(F))


def test_exact_sums_are_exact():
    # integer-valued products whose sums stay below 2^24 never round, whatever the order
    rng = np.random.default_rng(0)
    w = bits_np(rng.integers(-127, 128, (64, 512)).astype(F))
    x = bits_np(rng.integers(-127, 128, (3, 512)).astype(F))
    want = bf_np(x).astype(np.float64) @ bf_np(w).astype(np.float64).T
    assert np.array_equal(xp.mfma_gemm(w, x).astype(np.float64), want)


def test_within_fp32_chain_bound():
    rng = np.random.default_rng(1)
    w = _rand_bits(rng, (128, 1536), 0.02)
    x = _rand_bits(rng, (5, 1536))
    got = xp.mfma_gemm(w, x).astype(np.float64)
    a, b = bf_np(x).astype(np.float64), bf_np(w).astype(np.float64)
    want = a @ b.T
    # 192 roundings of the accumulator plus two truncations per group, each below 2^-23 of
    # the running magnitude
    bound = 3 * 192 * 2.0 ** -23 * (np.abs(a) @ np.abs(b).T)
    assert np.all(np.abs(got - want) <= bound)
    # and not a correctly rounded sum: the truncations are visible on long chains
    assert np.mean(got != want.astype(F)) > 0.01


def test_single_group_within_window_is_correctly_rounded():
    # products within 24 bits of the group maximum and a zero accumulator: the exact sum,
    # rounded once (round to nearest, ties to even)
    rng = np.random.default_rng(2)
    for _ in range(200):
        w = bits_np(((1 + rng.integers(0, 128, 8) / 128) * 2.0 ** rng.integers(-6, 1, 8)
                     * np.where(rng.random(8) < 0.5, -1, 1)).astype(F))
        x = bits_np(np.ones(8, F))
        exact_sum = float(np.sum(bf_np(w).astype(np.float64)))
        assert xp.mfma_chain(w, x) == F(exact_sum)


def test_truncation_and_tie_rules():
    one = bits_np(np.ones(8, F))
    # products below the group's 24-bit window are truncated toward zero: 1 + 2^-30 + ... = 1
    w = bits_np(np.array([1.0] + [2.0 ** -30] * 7, F))
    assert xp.mfma_chain(w, one) == F(1.0)
    # ... and a negative one is truncated toward zero too (not floored): 1 - tiny stays 1
    w = bits_np(np.array([1.0, -2.0 ** -30] + [0.0] * 6, F))
    assert xp.mfma_chain(w, one) == F(1.0)
    # an exact tie rounds to even: 1 + 2^-24 -> 1, 1 + 3 * 2^-24 -> 1 + 2^-22
    w = bits_np(np.array([1.0, 2.0 ** -24] + [0.0] * 6, F))
    assert xp.mfma_chain(w, one) == F(1.0)
    w = bits_np(np.array([1.0, 2.0 ** -23, 2.0 ** -24] + [0.0] * 5, F))
    assert xp.mfma_chain(w, one) == F(1.0 + 2.0 ** -22)
    # a group of zeros leaves the accumulator alone, including its low bits
    z = np.zeros(8, np.uint16)
    assert xp.mfma_chain(z, one, acc=F(1.0 + 2.0 ** -23)) == F(1.0 + 2.0 ** -23)


def test_exp2_det_accuracy_and_special_values():
    x = np.concatenate([np.linspace(-64, 0, 20001, dtype=F), -np.abs(np.random.default_rng(3).standard_normal(5000)
                                                                      * 8).astype(F)])
    x = x[x >= -64]
    got = xp.exp2_det(x).astype(np.float64)
    want = np.exp2(x.astype(np.float64))
    ulp = np.spacing(want.astype(F)).astype(np.float64)
    assert np.max(np.abs(got - want) / ulp) <= 3.0
    # exact powers of two (f = 0), the cut-off and -inf
    assert xp.exp2_det(np.array([0.0, -1.0, -17.0, -64.0], F)).tolist() == [1.0, 0.5, 2.0 ** -17, 2.0 ** -64]
    assert xp.exp2_det(np.array([-64.5, -np.inf, -1e30], F)).tolist() == [0.0, 0.0, 0.0]


def _flash_reference(q, keys, values, cap, p0, full, c, s):
    """FP32 softmax attention (Runtime.swift:389-444) with the kernel's key rotation."""
    T = q.shape[0]
    out = np.zeros((T, 16, 128), F)
    for t in range(T):
        pos = p0 + t
        first = 0 if full else max(0, pos - 2047)
        kp = np.arange(first, pos + 1)
        k = keys[kp % cap]
        if not full:
            base = max(0, p0 + (t // 16) * 16 - 2047)
            k = exact.rope_pair(k, c[kp - base], s[kp - base])
        sc = (torch.from_numpy(q[t]) @ torch.from_numpy(k).T) * torch.tensor(exact.SCALE)
        p = torch.softmax(sc, -1)
        out[t] = (p @ torch.from_numpy(values[kp % cap])).numpy()
    return roundbf_np(out)


@pytest.mark.parametrize("p0,tokens,cap,full", [
    (0, 20, 64, True),          # one partial tile
    (2040, 24, 2080, False),    # local: two chunk bases, window start inside the range
    (1100, 50, 1200, True),     # global: 18 tiles in three parts, merged
    (3000, 40, 2112, False),    # local: wrapped ring
])
def test_flash_twin_tracks_fp32_attention(p0, tokens, cap, full):
    rng = np.random.default_rng(p0 + tokens)
    q = roundbf_np(rng.standard_normal((tokens, 16, 128)).astype(F))
    keys = roundbf_np(rng.standard_normal((cap, 128)).astype(F))
    values = roundbf_np(rng.standard_normal((cap, 128)).astype(F))
    freqs = (10000.0 ** (-np.arange(64, dtype=np.float64) / 64)).astype(F)
    c, s = rope.local_table(freqs, rope.LOCAL_ROWS)
    got = bf_np(xp.flash(bits_np(q), bits_np(keys), bits_np(values), bits_np(c), bits_np(s), cap, p0, full))
    want = _flash_reference(q, keys, values, cap, p0, full, c, s).reshape(tokens, 2048)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-30))) - 7)
    diff = np.abs(got - want)
    assert np.all(diff <= ulp * 1.001 + 2.0 ** -14), float(diff.max())
    assert np.mean(diff > 0) < 0.01
    # a twin that dropped the newest key or shifted the window would disagree far more
    if not full:
        shifted = _flash_reference(q, keys, values, cap, p0 + 1, full, c, s).reshape(tokens, 2048)
        assert np.abs(shifted - got).max() > 0.05


def test_prefill_twin_tracks_decode_twin(oracle_weights, golden):
    # same model, same tokens: the prefill twin (MFMA order, flash softmax) and the decode
    # twin (GEMV order, split-K softmax) agree up to summation-order noise; the first
    # layer's keys, which only the qkv projection rounds, agree almost everywhere
    prompt = golden["config1"]["prompt"][:8]
    ex = exact.ExactDecoder(oracle_weights, 16, 16)
    bits, hidden, nxt = xp.ExactPrefill(ex).prefill(prompt)
    ex2 = exact.ExactDecoder(oracle_weights, 16, 16)
    for pos, t in enumerate(prompt):
        bits2, hidden2, nxt2 = ex2.step(t, pos)
    a, b = bf_np(bits).astype(np.float64), bf_np(bits2).astype(np.float64)
    assert np.sqrt(np.mean((a - b) ** 2)) < 0.03 and np.abs(a - b).max() < 0.15
    assert np.mean(ex.keys[0][:8] == ex2.keys[0][:8]) > 0.99
    assert np.array_equal(ex.values[0][:8] != 0, ex2.values[0][:8] != 0)


def test_chunked_prefill_twin_equals_one_call(oracle_weights, golden):
    # Runtime.prefill runs a prompt chunk by chunk (Runtime.swift:469-483).  Every prefill
    # operation acts on one token's row or on the keys that token sees, and the flash query
    # blocks of 8 tokens start at the same positions when chunks are multiples of 8, so the
    # twin over two 8-token chunks equals the twin over the whole prompt in every logit,
    # hidden and cached bit (a chunk placed at the wrong position, or keys of an earlier
    # chunk not seen, would not).  Both agree with the semantic oracle, which runs the
    # reference's 16-token chunks in torch order, within the measured summation-order noise
    # floor.
    from oracle import model as om
    prompt = golden["config1"]["prompt"][:16]
    runs = []
    for chunk in (2048, 8):
        ex = exact.ExactDecoder(oracle_weights, 32, 32)
        runs.append((xp.ExactPrefill(ex, chunk=chunk).prefill(prompt), ex))
    ((bits, hidden, nxt), ex0), ((b, h, t), ex) = runs
    assert np.array_equal(b, bits) and np.array_equal(h.view(np.uint32), hidden.view(np.uint32)) and t == nxt
    for layer in range(16):
        assert np.array_equal(ex.keys[layer], ex0.keys[layer]), layer
        assert np.array_equal(ex.values[layer], ex0.values[layer]), layer
    o = om.Oracle(oracle_weights, 32, dots="exact")
    o.prefill(prompt)
    ref = o.logits_fp32.numpy().astype(np.float64)
    err = np.abs(bf_np(bits).astype(np.float64) - ref)
    floor = golden["noise_floor"]["config1"]
    assert err.max() <= 1.5 * floor[0] and np.sqrt(np.mean(err ** 2)) <= 1.5 * floor[1], float(err.max())
    # a twin whose second chunk starts one position early caches different layer-1 keys
    ex = exact.ExactDecoder(oracle_weights, 32, 32)
    tw = xp.ExactPrefill(ex, chunk=8)
    tw.prefill(prompt[:8], kv_layers=2)
    tw.prefill(prompt[8:], p0=7, kv_layers=2)
    assert not np.array_equal(ex.keys[1][:16], ex0.keys[1][:16])
