"""QSA sparse global attention on the GPU (Runtime.swift:378-418, Kernels.metal:564-702) with
the synthetic seed-0 model and random-init indexers (synth.write_auxiliary).

* the selection kernel through plamo_kernel_qsa_select on the reference's known answers
  (QSATests.swift:6-46);
* QSATests.swift:48-70 restated: a budget that still covers every complete block
  (context 19, budget 16) and one above the context (budget 128) give the dense runtime's
  tokens and logits bit for bit, with the reference's counters;
* prefill (a chunk from position 0, then forwards starting inside blocks) and decode at
  budget 16, plain and .p12, equal the order-exact CPU twin (oracle/adapters.py QsaTwin on exact.ExactDecoder and
  exact_prefill.ExactPrefill) in every logit bit, the hidden row and the next token, and
  differ from dense attention;
* with MTP: a two-row sequential verification equals two scalar QSA forwards.
"""
import numpy as np
import pytest
import torch

import plamo_hip
from oracle import adapters as ad, exact, exact_prefill as xp
from plamo_hip import native

pytestmark = pytest.mark.gpu

INDEXER_BYTES = 2 * 2 * (640 * 1536 + 2 * 128)


def _rt(model_dir, context, budget=None, packed=False, mtp=False):
    d, sha = model_dir
    return plamo_hip.Runtime(d, context, packed=packed, source_sha256=sha, qsa_budget=budget, mtp=mtp)


def _kat_scores(visible, batch=3):
    blocks = (visible + batch - 1) // 4
    scores = np.zeros((batch, max(1, blocks)), np.float32)
    for t in range(batch):
        for b in range(blocks):
            scores[t, b] = np.float32(((b * 17 + t * 3) % 23) / 8) if b < (visible + t) // 4 else np.float32(1e9)
    return scores


def test_select_kernel_known_answers():
    lib = native.load()
    for visible in (1, 4, 7, 19, 64, 2051, 16387):
        for budget in (4, 16, 2048):
            scores = _kat_scores(visible)
            blocks = scores.shape[1]
            words = (blocks + 31) // 32
            sd = torch.from_numpy(scores).cuda()
            out = torch.full((3, words), -1, dtype=torch.int32, device="cuda")
            assert lib.plamo_kernel_qsa_select(sd.data_ptr(), blocks, 3, visible - 1, budget, out.data_ptr(), 0) == 0
            torch.cuda.synchronize()
            bits = out.cpu().numpy().view(np.uint32)
            for t in range(3):
                complete = (visible + t) // 4
                ranked = sorted(range(complete), key=lambda b: (-float(scores[t, b]), b))
                want = sorted(ranked[:budget // 4])
                got = [b for b in range(words * 32) if (bits[t, b >> 5] >> (b & 31)) & 1]
                assert got == want, (visible, budget, t)
    print("  qsa_select: every known answer of the reference's selection test", flush=True)


def test_select_kernel_rejects_bad_shapes():
    lib = native.load()
    x = torch.zeros(64, dtype=torch.float32, device="cuda")
    for blocks, tokens, start in ((0, 1, 0), (8193, 1, 0), (4, 0, 0), (4, 1, -1), (4, 3, 17)):
        assert lib.plamo_kernel_qsa_select(x.data_ptr(), blocks, tokens, start, 16, x.data_ptr(), 0) != 0


def test_visible_tail_keeps_all_keys(model_dir):
    # QSATests.swift:48-58
    dense, sparse = _rt(model_dir, 19, packed=True), _rt(model_dir, 19, 16, packed=True)
    try:
        ids = [1] + list(range(500, 517))
        assert dense.prefill(ids) == sparse.prefill(ids)
        assert np.array_equal(dense.logit_bits(), sparse.logit_bits())
        st = sparse.stats()
        assert st["sparse_queries"] > 0 and st["sparse_keys"] == st["dense_keys"]
        assert st["auxiliary_bytes"] == INDEXER_BYTES
    finally:
        dense.close()
        sparse.close()


def test_dense_budget_matches_original(model_dir):
    # QSATests.swift:60-69
    dense, sparse = _rt(model_dir, 64, packed=True), _rt(model_dir, 64, 128, packed=True)
    try:
        ids = [1, 500, 600, 700, 800]
        assert dense.prefill(ids) == sparse.prefill(ids)
        assert np.array_equal(dense.logit_bits(), sparse.logit_bits())
        assert sparse.stats()["sparse_queries"] == 0
    finally:
        dense.close()
        sparse.close()


def _counts(calls, budget):
    # Runtime.swift:396-402 per global layer (two of them)
    q = s = d = 0
    for p0, n in calls:
        if p0 + n <= budget:
            continue
        for t in range(n):
            v = p0 + t + 1
            q, d, s = q + 2, d + 2 * v, s + 2 * (min(v // 4, budget // 4) * 4 + v % 4)
    return q, s, d


@pytest.mark.parametrize("packed", [False, True])
def test_prefill_and_decode_bit_exact(model_dir, oracle_weights, packed):
    context, budget = 160, 16
    rng = np.random.default_rng(31)
    prompt = [1] + rng.integers(1024, 107520, 69).tolist()
    adapters = ad.Adapters(model_dir[0])
    rt, dense = _rt(model_dir, context, budget, packed=packed), _rt(model_dir, context, packed=packed)
    try:
        # a prompt, then forwards of 16 and 13 rows starting inside blocks 10 and 14
        rt.prefill(prompt[:41])
        rt.forward(prompt[41:57])
        nxt = rt.forward(prompt[57:])
        dense.prefill(prompt[:41])
        dense.forward(prompt[41:57])
        dense.forward(prompt[57:])
        assert not np.array_equal(rt.logit_bits(), dense.logit_bits())
        ex = exact.ExactDecoder(oracle_weights, context, rt.stats()["local_capacity"],
                                qsa=ad.QsaTwin(adapters, context, budget))
        pre = xp.ExactPrefill(ex)
        pre.prefill(prompt[:41])
        pre.prefill(prompt[41:57], p0=41)
        bits, hidden, want = pre.prefill(prompt[57:], p0=57)
        assert np.array_equal(rt.logit_bits(), bits)
        assert np.array_equal(rt.hidden().view(np.uint32), hidden.view(np.uint32))
        assert nxt == want
        print(f"  QSA prefill of 41 + 16 + 13 tokens (budget {budget}, packed={packed}): bit-exact, next {nxt}",
              flush=True)
        # the prompt's counters follow Runtime.fill's 16-row forwards (Runtime.swift:476)
        calls = [(0, 16), (16, 16), (32, 9), (41, 16), (57, 13)]
        pos, t = len(prompt), nxt
        for _ in range(10):
            got = rt.forward([t])
            bits, hidden, want = ex.step(t, pos)
            assert np.array_equal(rt.logit_bits(), bits), pos
            assert np.array_equal(rt.hidden().view(np.uint32), hidden.view(np.uint32)), pos
            assert got == want, pos
            calls.append((pos, 1))
            pos, t = pos + 1, got
        print(f"  QSA decode to position {pos}: bit-exact", flush=True)
        st = rt.stats()
        assert (st["sparse_queries"], st["sparse_keys"], st["dense_keys"]) == _counts(calls, budget)
    finally:
        rt.close()
        dense.close()


def test_verification_rows_with_qsa(model_dir):
    context, budget = 96, 16
    prefix = [1] + [500 + 7 * k for k in range(44)]
    scalar = _rt(model_dir, context, budget, mtp=True)
    batched = _rt(model_dir, context, budget, mtp=True)
    try:
        assert scalar.prefill(prefix) == batched.prefill(prefix)
        expected, nxt = [], []
        for t in (600, 700):
            nxt.append(scalar.forward([t]))
            expected.append(scalar.logit_bits())
        batched.forward([600, 700], all=True, sequential=True)
        assert batched.predictions() == nxt
        for i in range(2):
            assert np.array_equal(batched.logit_bits(i), expected[i]), i
        batched.rewind(len(prefix) + 2, 1)
        assert batched.forward([901]) == scalar.forward([901])
        assert np.array_equal(batched.logit_bits(), scalar.logit_bits())
        assert batched.stats()["sparse_keys"] == scalar.stats()["sparse_keys"]
    finally:
        scalar.close()
        batched.close()
