"""MTP on the GPU (Runtime.draft / forward(all:sequential:) / rewind, Runtime.swift:322-538)
with the synthetic seed-0 model and random-init adapters (synth.write_auxiliary).

* the draft equals the order-exact CPU restatement (oracle/adapters.py) in every logit bit
  and its token, plain and .p12, also after a verification pass and a rewind;
* VerificationTests.swift:6-53: a two-row sequential verification (one pass of the
  multi-row kernels over the weights, the reference's linear_pair pass) equals two scalar
  forwards bit for bit (every row's logits, hidden row and prediction), pass after pass;
  three rows are refused without touching the state, rewind keeps the chosen row and
  continues like a clean runtime;
* VerificationTests.swift:96-108 (draft shapes and refusals), LogitsTests.swift:49-68 (rows
  of a non-sequential two-row forward and rewind to the second row).
"""
import numpy as np
import pytest

import plamo_hip
from oracle import adapters as ad, exact

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def adapters(model_dir):
    return ad.Adapters(model_dir[0])


def _mtp(model_dir, context, packed=False, qsa_budget=None):
    d, sha = model_dir
    return plamo_hip.Runtime(d, context, packed=packed, source_sha256=sha, mtp=True, qsa_budget=qsa_budget)


@pytest.mark.parametrize("packed", [False, True])
def test_draft_bit_exact(model_dir, oracle_weights, adapters, packed):
    prefix = [1] + [500 + k % 37 for k in range(31)]
    rt = _mtp(model_dir, 64, packed)
    try:
        nxt = rt.prefill(prefix)
        ex = exact.ExactDecoder(oracle_weights, 16, 16)
        for first in (nxt, 500, 107519):
            before = rt.position
            got = rt.draft(first)
            bits, tok = ad.mtp_draft(ex, adapters, rt.hidden(), first)
            assert got == [tok], (packed, first)
            assert rt.position == before and rt.predictions() == [tok]
            print(f"  packed={packed} draft after {first}: {tok}, bit-exact", flush=True)
        st = rt.stats()
        assert st["auxiliary_bytes"] == 2 * (256 * 3072 + 1536 * 256)
    finally:
        rt.close()


def _bits(rt, slot=0):
    return rt.logit_bits(slot).copy()


@pytest.mark.parametrize("packed", [False, True])
def test_batched_verification_and_rollback(model_dir, packed):
    # VerificationTests.swift:17-53 (length 31, no QSA budget)
    length = 31
    prefix = [1] + [500 + k % 37 for k in range(length - 1)]
    scalar, batched = _mtp(model_dir, length + 32, packed), _mtp(model_dir, length + 32, packed)
    try:
        assert scalar.prefill(prefix) == batched.prefill(prefix)
        before = _bits(batched)
        for all_, seq in ((True, False), (False, True), (True, True)):
            with pytest.raises(plamo_hip.PlamoError, match="Invalid tokens or context exhausted"):
                batched.forward([600, 700, 800], all=all_, sequential=seq)
            assert batched.position == length
            assert np.array_equal(_bits(batched), before)
        inputs = [600, 700]
        expected, nxt = [], []
        for t in inputs:
            nxt.append(scalar.forward([t]))
            expected.append(_bits(scalar))
        batched.forward(inputs, all=True, sequential=True)
        assert batched.predictions() == nxt
        for i in range(2):
            assert np.array_equal(_bits(batched, i), expected[i]), i
        batched.rewind(length + 2, 1)
        assert batched.position == length + 2 and batched.predictions() == [nxt[1]]
        assert np.array_equal(_bits(batched), expected[1])
        assert batched.forward([901]) == scalar.forward([901])
        assert np.array_equal(_bits(batched), _bits(scalar))
        batched.reset()
        batched.prefill(prefix)
        batched.forward(inputs, all=True, sequential=True)
        batched.rewind(length + 1, 0)
        clean = _mtp(model_dir, length + 32, packed)
        try:
            clean.prefill(prefix)
            clean.forward([inputs[0]])
            assert batched.forward([901]) == clean.forward([901])
            assert np.array_equal(_bits(batched), _bits(clean))
            assert np.array_equal(batched.hidden().view(np.uint32), clean.hidden().view(np.uint32))
        finally:
            clean.close()
        with pytest.raises(plamo_hip.PlamoError, match="Invalid verification rollback"):
            batched.rewind(0, 9)
        print(f"  packed={packed}: verification rows equal scalar forwards, rewinds continue cleanly", flush=True)
    finally:
        scalar.close()
        batched.close()


def test_draft_after_rollback_bit_exact(model_dir, oracle_weights, adapters):
    # the draft reads the kept row's hidden state: after verifying two rows and keeping the
    # first, it equals the twin's draft from that row
    prefix = [1] + list(range(500, 532))
    rt = _mtp(model_dir, 64)
    try:
        rt.prefill(prefix)
        rt.forward([600, 700], all=True, sequential=True)
        h0 = None
        rt.rewind(rt.position - 1, 0)
        h0 = rt.hidden()
        ex = exact.ExactDecoder(oracle_weights, 16, 16)
        bits, tok = ad.mtp_draft(ex, adapters, h0, 800)
        assert rt.draft(800) == [tok]
        assert rt.position == len(prefix) + 1
    finally:
        rt.close()


def test_trained_draft_shapes(model_dir):
    # VerificationTests.swift:96-108
    rt = _mtp(model_dir, 64, packed=True)
    try:
        with pytest.raises(plamo_hip.PlamoError, match="MTP requires a prefetched context and trained adapters"):
            rt.draft(500)
        rt.prefill([1, 500, 600])
        for token in (-1, 107520, 1, 16):
            with pytest.raises(plamo_hip.PlamoError, match="MTP requires"):
                rt.draft(token)
        before = rt.position
        drafts = rt.draft(500)
        assert len(drafts) == 1 and 0 <= drafts[0] < 107520 and rt.position == before
    finally:
        rt.close()
    d, sha = model_dir
    plain = plamo_hip.Runtime(d, 64, source_sha256=sha)
    try:
        plain.prefill([1, 500, 600])
        with pytest.raises(plamo_hip.PlamoError, match="MTP requires"):
            plain.draft(500)
        with pytest.raises(plamo_hip.PlamoError, match="Invalid tokens or context exhausted"):
            plain.forward([600, 700], all=True, sequential=True)
    finally:
        plain.close()


@pytest.mark.parametrize("packed", [False, True])
def test_matrix_rows_and_rewind(model_dir, packed):
    # LogitsTests.swift:49-68: a non-sequential two-row forward outputs both rows
    rt = _mtp(model_dir, 64, packed)
    try:
        rt.prefill([1] + list(range(500, 532)))
        rt.forward([600, 700], all=True)
        ids = rt.predictions()
        assert len(ids) == 2
        rows = [rt.logits(i) for i in range(2)]
        for i in range(2):
            assert np.all(np.isfinite(rows[i]))
            assert ids[i] == int(np.argmax(rows[i]))
        rt.rewind(rt.position, 1)
        assert rt.predictions() == [ids[1]]
        assert np.array_equal(rt.logits().view(np.uint32), rows[1].view(np.uint32))
    finally:
        rt.close()


def test_batch_refuses_adapters(model_dir):
    # Batch.swift:34-36: dense greedy inference only
    rt = _mtp(model_dir, 64)
    try:
        with pytest.raises(plamo_hip.PlamoError, match="Batch requires dense greedy inference"):
            plamo_hip.Batch(rt)
    finally:
        rt.close()


@pytest.mark.parametrize("packed", [False, True])
def test_repeated_verifications_equal_scalar_steps(model_dir, packed):
    # the two-row verification pass (one read of the weights for both rows, replayed from a
    # captured graph) equals two scalar steps in every logit and hidden bit, replay after
    # replay, with rewinds, host synchronisations and single steps between the replays
    prefix = [1] + [300 + 11 * k for k in range(40)]
    pair, scalar = _mtp(model_dir, 128, packed), _mtp(model_dir, 128, packed)
    try:
        assert pair.prefill(prefix) == scalar.prefill(prefix)
        rng = np.random.default_rng(4)
        for it in range(5):
            cand = [int(t) for t in rng.integers(1024, 107520, 2)]
            pair.forward(cand, all=True, sequential=True)
            want, nxt = [], []
            for t in cand:
                nxt.append(scalar.forward([t]))
                want.append((_bits(scalar), scalar.hidden().view(np.uint32).copy()))
            assert pair.predictions() == nxt, it
            for i in range(2):
                assert np.array_equal(_bits(pair, i), want[i][0]), (it, i)
            pair.rewind(pair.position, 1)
            assert np.array_equal(pair.hidden().view(np.uint32), want[1][1]), it
            t = int(rng.integers(1024, 107520))
            assert pair.forward([t]) == scalar.forward([t]), it
            assert np.array_equal(_bits(pair), _bits(scalar)), it
        print(f"  packed={packed}: five verification passes equal scalar steps", flush=True)
    finally:
        pair.close()
        scalar.close()
