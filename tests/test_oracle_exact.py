"""Pins of the order-exact decode restatement (oracle/exact.py) on the CPU."""
import os

import numpy as np
import pytest
import torch

from oracle import exact, model as om
from oracle.bf16 import bf_np, bits_np, roundbf_np

FIXTURE_DOT2 = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "dot2_accumulate.npz")


def test_exp_det_accuracy():
    x = np.concatenate([np.linspace(-79.9, 88.7, 200001, dtype=np.float32),
                        np.float32(np.random.default_rng(0).standard_normal(100000) * 10)]).astype(np.float32)
    got = exact.exp_det(x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - want) / ulp) <= 2.0
    assert exact.exp_det(np.array([-np.inf, -80.5, 0.0, 100.0], np.float32)).tolist() == [0.0, 0.0, 1.0, np.inf]


def test_gemv_order_is_a_valid_fp32_sum():
    rng = np.random.default_rng(1)
    w = bf_np(np.float32(rng.standard_normal((64, 1536)) * 0.02).view(np.uint32) >> 16)
    x = bf_np(np.float32(rng.standard_normal(1536)).view(np.uint32) >> 16)
    got = exact.gemv(w, x).astype(np.float64)
    want = w.astype(np.float64) @ x.astype(np.float64)
    bound = 1536 * 2 ** -24 * (np.abs(w).astype(np.float64) @ np.abs(x).astype(np.float64))
    assert np.all(np.abs(got - want) <= bound)


def _pairs(lo, hi):
    return (bits_np(np.asarray(lo, np.float32)).astype(np.uint32)
            | (bits_np(np.asarray(hi, np.float32)).astype(np.uint32) << 16))


def test_dot2_model_reproduces_device_accumulators():
    # the device is the authority for v_dot2_f32_bf16 rounding: every recorded accumulator,
    # bit for bit, by the general fold and by the fast form the GEMV restatement uses
    from golden import make_dot2_fixture as mk
    rec = np.load(FIXTURE_DOT2)
    for name, (a, b, c) in mk.cases().items():
        for fast in (True, False):
            got = mk.stored(name, exact.dot2_chain(a, b, c, fast=fast))
            for key, want in got.items():
                bad = int(np.sum(want.view(np.uint32) != rec[key].view(np.uint32)))
                assert bad == 0, (key, fast, bad)


def test_dot2_rules():
    one = np.float32(1.0)
    # a product below the 24-bit window of the larger one is truncated toward zero
    assert exact.dot2_chain(_pairs([[1.0]], [[2.0 ** -30]]), _pairs([[1.0]], [[1.0]]), [0.0])[0, 0] == one
    # the window is set by the products, not by the accumulator: 1 - 1 + 2^-30 = 0
    assert exact.dot2_chain(_pairs([[1.0]], [[-1.0]]), _pairs([[1.0]], [[1.0]]), [2.0 ** -30])[0, 0] == 0.0
    # the sum is floored 31 bits below its leading bit before the rounding: a tie with a
    # sticky bit below that window rounds to even, 1 + 2^-24 + 2^-40 -> 1
    assert exact.dot2_chain(_pairs([[2.0 ** -12]], [[2.0 ** -20]]), _pairs([[2.0 ** -12]], [[2.0 ** -20]]),
                            [1.0])[0, 0] == one
    # ... while a sticky bit inside it rounds up: 1 + 2^-24 + 2^-30 -> 1 + 2^-23
    assert exact.dot2_chain(_pairs([[2.0 ** -12]], [[2.0 ** -15]]), _pairs([[2.0 ** -12]], [[2.0 ** -15]]),
                            [1.0])[0, 0] == np.float32(1 + 2.0 ** -23)
    # zero products leave the accumulator and its low bits unchanged
    acc = np.float32(1 + 2.0 ** -23)
    assert exact.dot2_chain(_pairs([[0.0]], [[0.0]]), _pairs([[3.0]], [[5.0]]), [acc])[0, 0] == acc
    # products inside one window and a zero accumulator: the exact sum, rounded once
    rng = np.random.default_rng(4)
    a = roundbf_np(rng.standard_normal((1, 2000, 2)).astype(np.float32))
    b = roundbf_np(rng.standard_normal((1, 2000, 2)).astype(np.float32))
    got = exact.dot2_chain(_pairs(a[..., 0], a[..., 1]), _pairs(b[..., 0], b[..., 1]), np.zeros(2000, np.float32))
    want = (a[..., 0].astype(np.float64) * b[..., 0] + a[..., 1].astype(np.float64) * b[..., 1]).astype(np.float32)
    close = np.abs(np.log2(np.abs(a[..., 0] * b[..., 0]) + 1e-30) - np.log2(np.abs(a[..., 1] * b[..., 1]) + 1e-30)) < 8
    assert np.array_equal(got[close], want[close])


def test_gemv_is_lane_chains_of_dot2():
    # a row whose only nonzero columns are lane l's (it * 512 + 8 l .. +8) returns lane l's
    # chain: four dot2 steps per column block, pairs in column order, blocks in order
    rng = np.random.default_rng(3)
    n = 1536
    x = roundbf_np(rng.standard_normal(n).astype(np.float32))
    w = np.zeros((64, n), np.float32)
    for l in range(64):
        for it in range(3):
            w[l, it * 512 + 8 * l:it * 512 + 8 * l + 8] = roundbf_np(
                rng.standard_normal(8).astype(np.float32) * 2.0 ** rng.integers(-12, 4))
    got = exact.gemv(w, x)
    for l in (0, 1, 31, 63):
        cols = np.concatenate([np.arange(it * 512 + 8 * l, it * 512 + 8 * l + 8) for it in range(3)])
        a = _pairs(w[l, cols[0::2]], w[l, cols[1::2]])[:, None]
        b = _pairs(x[cols[0::2]], x[cols[1::2]])[:, None]
        chain = exact.dot2_chain(a, b, [0.0], fast=False)[-1, 0]
        assert got[l] == chain, l


def test_attention_scores_are_dot2_chains():
    # each raw score: four 32-dim chains of dot2 steps over the dim pairs in order, summed as
    # (c0 + c1) + (c2 + c3); checked against the general fold one chain at a time
    rng = np.random.default_rng(6)
    q = roundbf_np(rng.standard_normal((16, 128)).astype(np.float32))
    k = roundbf_np((rng.standard_normal((70, 128)) * 2.0 ** rng.integers(-6, 6, (70, 1))).astype(np.float32))
    got = exact.attn_scores(q, k)
    for h, j in ((0, 0), (5, 17), (15, 69)):
        chains = []
        for c in range(4):
            d = np.arange(32 * c, 32 * c + 32)
            a = _pairs(q[h, d[0::2]], q[h, d[1::2]])[:, None]
            b = _pairs(k[j, d[0::2]], k[j, d[1::2]])[:, None]
            chains.append(exact.dot2_chain(a, b, [0.0], fast=False)[-1, 0])
        assert got[h, j] == (chains[0] + chains[1]) + (chains[2] + chains[3]), (h, j)
    # small integers: every sum exact, whatever the order
    qi = rng.integers(-8, 9, (16, 128)).astype(np.float32)
    ki = rng.integers(-8, 9, (5, 128)).astype(np.float32)
    assert np.array_equal(exact.attn_scores(qi, ki), (qi.astype(np.float64) @ ki.T.astype(np.float64)).astype(np.float32))


def test_attention_pv_is_fma_chains():
    # per head and dim: keys 0..31 and 32..nk-1 as two chains of fused multiply-adds from 0
    # (one rounding per step: exact in float64 for these magnitudes), then the halves added
    rng = np.random.default_rng(8)
    nk = 45
    e = np.zeros((16, 64), np.float32)
    e[:, :nk] = rng.uniform(0.1, 1.0, (16, nk)).astype(np.float32)
    v = roundbf_np(rng.uniform(-2, 2, (nk, 128)).astype(np.float32))
    got = exact.attn_pv(e, bits_np(v))
    fused = np.zeros((16, 128), np.float32)
    unfused = np.zeros((16, 128), np.float32)
    for hf, ks in enumerate((range(0, 32), range(32, nk))):
        a = np.zeros((16, 128), np.float32)
        b = np.zeros((16, 128), np.float32)
        for j in ks:
            a = (a.astype(np.float64) + e[:, j:j + 1].astype(np.float64) * v[j].astype(np.float64)).astype(np.float32)
            b = (b + (e[:, j:j + 1] * v[j]).astype(np.float32)).astype(np.float32)
        fused = (fused + a).astype(np.float32) if hf else a
        unfused = (unfused + b).astype(np.float32) if hf else b
    assert np.array_equal(got, fused)
    assert not np.array_equal(got, unfused)


def test_block_sumsq_and_norm():
    v = np.full(1536, 2.0, np.float32)
    assert exact.block_sumsq(v) == np.float32(6144.0)
    z = exact.norm_rows(v, np.zeros(1536, np.uint16), 1.0)
    assert np.all(z == 1.0)


@pytest.mark.slow
def test_exact_decoder_tracks_semantic_oracle(oracle_weights, golden):
    # same algorithm, different summation order: agreement within the measured noise floor
    prompt = golden["config1"]["prompt"][:6]
    ex = exact.ExactDecoder(oracle_weights, 16, 16)
    o = om.Oracle(oracle_weights, 16)
    for pos, t in enumerate(prompt):
        bits, _, nxt = ex.step(t, pos)
        o.forward([t])
    ref = o.logits_fp32.numpy().astype(np.float64)
    got = bf_np(bits).astype(np.float64)
    rmse = float(np.sqrt(np.mean((got - ref) ** 2)))
    assert rmse < 0.03 and np.argmax(got) == np.argmax(ref)


def _attention_pair(context, cap_local, seed):
    """An ExactDecoder and a semantic Oracle that share only attention state (keys, values,
    norm gains, RoPE tables): no model weights are needed for `attention`/`_attention`."""
    from oracle import rope
    rng = np.random.default_rng(seed)
    f_local, f_full = rope.synthetic_frequencies()
    ex = exact.ExactDecoder.__new__(exact.ExactDecoder)
    ex.context = context
    ex.cap = [context if i % 8 == 7 else cap_local for i in range(16)]
    qn = exact.bits_np((rng.standard_normal(128) * 0.1).astype(np.float32))
    kn = exact.bits_np((rng.standard_normal(128) * 0.1).astype(np.float32))
    ex.layers = [{"q_norm": qn, "k_norm": kn} for _ in range(16)]
    ex.lc, ex.ls = rope.local_table(f_local, 2064)
    ex.gc, ex.gs = rope.global_table(f_full, context)
    ex.keys = [exact.bits_np(rng.standard_normal((c, 128)).astype(np.float32)) for c in ex.cap]
    ex.values = [exact.bits_np(rng.standard_normal((c, 128)).astype(np.float32)) for c in ex.cap]
    o = om.Oracle.__new__(om.Oracle)
    o.dots = "exact"  # correctly rounded dot products: the same on every machine
    o.context = context
    o.capacity = list(ex.cap)
    o.local = (torch.from_numpy(ex.lc), torch.from_numpy(ex.ls))
    o.glob = (torch.from_numpy(ex.gc), torch.from_numpy(ex.gs))
    return ex, o, qn, kn, rng


def _semantic_row(ex, o, layer, qkv, pos, qn):
    """The semantic oracle's attention for the same row after the twin wrote the new key."""
    full = layer % 8 == 7
    o.keys = [torch.from_numpy(k.astype(np.int32)) for k in ex.keys]
    o.values = [torch.from_numpy(v.astype(np.int32)) for v in ex.values]
    z = om.norm(torch.from_numpy(qkv[:2048].reshape(16, 128)), torch.from_numpy(qn.astype(np.int32)), 1.0)
    base = 0 if full else max(0, pos - 2047)
    c, s = (o.glob[0][pos], o.glob[1][pos]) if full else (o.local[0][pos - base], o.local[1][pos - base])
    q = om.rotate(z, c, s)
    return o._attention(layer, q[None], 1, pos)[0].numpy()


@pytest.mark.parametrize("layer,pos,context,cap_local", [
    (0, 4090, 8192, 2064),    # local: window base 2043, the 2064-slot ring wrapped, 32 partitions
    (3, 2047, 4096, 2064),    # local: the window exactly fills from key 0
    (7, 5000, 8192, 2064),    # global: 79 partitions (> 64: the attn_merge_kernel order)
    (15, 32767, 32768, 2064), # global at the context cap: 512 partitions
])
def test_exact_attention_tracks_semantic_past_the_window(layer, pos, context, cap_local):
    # ExactDecoder.attention (the GPU's order-exact twin) against the semantic oracle's
    # _attention (pinned by closed forms) where the twin's window, ring, RoPE base and
    # partition-merge logic matter: same BF16 result but for summation-order rounding.
    ex, o, qn, kn, rng = _attention_pair(context, cap_local, layer + pos)
    qkv = exact.bf_np(exact.bits_np(rng.standard_normal(2304).astype(np.float32)))
    got = ex.attention(layer, qkv, pos)
    want = _semantic_row(ex, o, layer, qkv, pos, qn)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-30))) - 7)
    diff = np.abs(got - want)
    assert np.all(diff <= ulp * 1.001 + 2.0 ** -20), float(diff.max())
    assert np.mean(diff > 0) < 0.02, float(np.mean(diff > 0))
    # a dropped key or a wrong window would move far more than an ulp: the same row with the
    # window shifted by one key disagrees grossly
    if layer % 8 != 7:
        o2 = om.Oracle.__new__(om.Oracle)
        o2.__dict__.update(o.__dict__)
        shifted = _semantic_row(ex, o2, layer, qkv, pos - 1, qn) if pos > 2047 else None
        if shifted is not None:
            assert np.abs(shifted - got).max() > 16 * np.abs(got - want).max()


@pytest.mark.parametrize("layer,start,base,cap", [(0, 4090, 2043, 2064), (7, 65, 0, 67)])
def test_exact_attention_window_mean(layer, start, base, cap):
    # PlamoTests.swift:156-194 restated on the twin: zero queries score every visible key 0,
    # so each output is the mean of the visible values (value of position p: p % 17 - 8)
    ex, o, qn, kn, rng = _attention_pair(cap if layer % 8 == 7 else 8192, cap, 5)
    for p in range(base, start + 2):
        ex.values[layer][p % cap] = exact.bits_np(np.float32(p % 17 - 8))
    for pos in (start, start + 1):
        qkv = np.zeros(2304, np.float32)
        qkv[2176:] = np.float32(pos % 17 - 8)
        got = ex.attention(layer, qkv, pos)
        begin = 0 if layer % 8 == 7 else pos - 2047
        want = sum(k % 17 - 8 for k in range(begin, pos + 1)) / (pos - begin + 1)
        assert np.all(np.abs(got - want) <= 3e-4), (pos, want, got[0])
