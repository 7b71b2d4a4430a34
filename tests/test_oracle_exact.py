"""Pins of the order-exact decode restatement (oracle/exact.py) on the CPU."""
import numpy as np
import pytest
import torch

from oracle import exact, model as om
from oracle.bf16 import bf_np


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


def test_c_and_numpy_gemv_agree():
    if exact._c_lib() is None:
        pytest.skip("oracle C restatement not built (make -C oracle)")
    rng = np.random.default_rng(2)
    w = bf_np(np.float32(rng.standard_normal((300, 6144)) * 0.02).view(np.uint32) >> 16)
    x = bf_np(np.float32(rng.standard_normal(6144)).view(np.uint32) >> 16)
    assert np.array_equal(exact.gemv(w, x).view(np.uint32), exact.gemv_numpy(w, x).view(np.uint32))


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
