"""QSA block selection on the CPU: the order-exact indexer restatement (oracle/adapters.py
QsaTwin, exact_flash.c's key mask, ExactDecoder's masked attention) pinned against

* the reference's selection known-answer test (QSATests.swift:6-46: visible 1 .. 16387,
  budgets 4 / 16 / 2048, three query rows, scores ((17 b + 3 t) % 23) / 8 with ties, and
  1e9 past the complete blocks), with a tie-order mistake planted to show the check sees it;
* FP64 textbook indexer scores (mean of four raw keys, head RMSNorm with gain w + 1, global
  RoPE at the block's first position, sum of ReLU'd head dot products / sqrt(128)) within
  the rounding of its BF16 steps, with mistakes planted in the textbook (no ReLU, gain w,
  block keys rotated at 4b + 1) each outside that bound;
* the masked prefill attention against an FP64 softmax over the selected keys, and an
  all-selected mask bit-equal to no mask;
* the decode twin: a small budget equals a covering one until the first query sees more
  complete blocks than the budget allows, and differs later.
"""
import types

import numpy as np
import pytest

from oracle import adapters as ad, exact, exact_prefill as xp, rope
from oracle.bf16 import bf_np, bits_np, roundbf_np

F = np.float32


def _kat_scores(visible, batch=3):
    blocks = (visible + batch - 1) // 4
    scores = np.zeros((batch, max(1, blocks)), F)
    for t in range(batch):
        for b in range(blocks):
            scores[t, b] = F(((b * 17 + t * 3) % 23) / 8) if b < (visible + t) // 4 else F(1e9)
    return scores


def _kat_expected(scores_row, complete, budget):
    # QSATests.swift:33-38: rank by score descending, ties to the lower index, first budget/4
    ranked = sorted(range(complete), key=lambda b: (-float(scores_row[b]), b))
    return sorted(ranked[:budget // 4])


KAT_CASES = [(v, b) for v in (1, 4, 7, 19, 64, 2051, 16387) for b in (4, 16, 2048)]


def test_selection_known_answers():
    for visible, budget in KAT_CASES:
        scores = _kat_scores(visible)
        for t in range(3):
            complete = (visible + t) // 4
            got = np.flatnonzero(ad.select(scores[t], complete, budget)).tolist()
            assert got == _kat_expected(scores[t], complete, budget), (visible, budget, t)
            # the attended keys: the chosen blocks' four keys, then the unfinished block's
            keys = [4 * b + i for b in got for i in range(4)] + list(range(4 * complete, visible + t))
            assert len(keys) == min(complete, budget // 4) * 4 + (visible + t) % 4
            assert all(k < visible + t for k in keys)


def test_selection_tie_order_is_checked():
    # a selection that breaks ties toward the higher index fails the known answers
    def higher_ties(row, complete, budget):
        k = min(complete, budget // 4)
        ranked = sorted(range(complete), key=lambda b: (-float(row[b]), -b))
        return sorted(ranked[:k])

    failed = 0
    for visible, budget in KAT_CASES:
        scores = _kat_scores(visible)
        for t in range(3):
            complete = (visible + t) // 4
            failed += higher_ties(scores[t], complete, budget) != _kat_expected(scores[t], complete, budget)
    assert failed > 0


def test_selection_negative_scores_clamp():
    # values compare as max(score, 0): negative scores tie with zero at the lower index
    s = np.array([-3.0, 0.5, -1.0, 0.0, 2.0], F)
    assert np.flatnonzero(ad.select(s, 5, 8)).tolist() == [1, 4]
    assert np.flatnonzero(ad.select(s, 5, 12)).tolist() == [0, 1, 4]
    assert ad.select(s, 5, 20).all() and ad.select(s, 5, 2048).all()


@pytest.fixture(scope="module")
def indexer_case():
    rng = np.random.default_rng(3)
    ctx = 64
    gc, gs = rope.global_table(rope.synthetic_frequencies()[1], ctx)
    ex = types.SimpleNamespace(gc=gc, gs=gs)
    A = types.SimpleNamespace(qsa={7: {"proj": np.zeros((640, 1536), np.uint16),
                                       "q_norm": bits_np(rng.normal(0, 0.3, 128).astype(F)),
                                       "k_norm": bits_np(rng.normal(0, 0.3, 128).astype(F))}})
    rows = roundbf_np(rng.normal(0, 1, (40, 640)).astype(F))
    return ex, A, rows


def _max_error(a, b):
    return max((float(np.max(np.abs(np.asarray(x, np.float64) - y))) for x, y in zip(a, b) if len(y)), default=0.0)


def test_indexer_scores_match_textbook(indexer_case):
    ex, A, rows = indexer_case
    tw = ad.QsaTwin(A, 64, 16)
    tw._rows(ex, 7, rows, 0)
    ref = ad.textbook_scores(A, 7, ex.gc, ex.gs, rows)
    scale = max(float(np.max(np.abs(r))) for r in ref if len(r))
    tol = 0.012 * scale  # BF16 queries and block keys: ~2^-8 relative each
    err = _max_error(tw.last_scores[7], ref)
    print(f"  indexer scores: max |twin - textbook| {err:.4f}, bound {tol:.4f}")
    assert err <= tol
    for name, kw in (("no ReLU", {"relu": False}), ("gain w", {"gain_offset": 0.0}),
                     ("block keys at 4b + 1", {"k_rope_shift": 1})):
        planted = ad.textbook_scores(A, 7, ex.gc, ex.gs, rows, **kw)
        perr = _max_error(tw.last_scores[7], planted)
        print(f"  planted {name}: {perr:.4f}")
        assert perr > 4 * tol, name


def test_indexer_state_across_calls(indexer_case):
    # a prefill chunk and the same rows one by one (decode) build the same block keys and masks
    ex, A, rows = indexer_case
    whole, steps = ad.QsaTwin(A, 64, 8), ad.QsaTwin(A, 64, 8)
    m_whole = whole._rows(ex, 7, rows[:37], 0)
    m_steps = np.concatenate([steps._rows(ex, 7, rows[p:p + 1], p) for p in range(37)])
    assert np.array_equal(m_whole, m_steps)
    assert np.array_equal(whole.pooled[7], steps.pooled[7]) and np.array_equal(whole.raw[7], steps.raw[7])
    # a chunk starting inside a block completes it from keys of the previous call
    split = ad.QsaTwin(A, 64, 8)
    m_split = np.concatenate([split._rows(ex, 7, rows[:13], 0), split._rows(ex, 7, rows[13:37], 13)])
    assert np.array_equal(m_split, m_whole) and np.array_equal(split.pooled[7], whole.pooled[7])
    # selection sizes: min(complete, 2) blocks per query
    for t in range(37):
        assert int(sum(bin(int(w)).count("1") for w in m_whole[t])) == min((t + 1) // 4, 2)


def _softmax_ref(q, k, v, seen):
    s = (q.astype(np.float64) @ k.astype(np.float64).T) / np.sqrt(128)
    s = np.where(seen, s, -np.inf)
    p = np.exp(s - s.max())
    return (p / p.sum()) @ v.astype(np.float64)


def test_masked_flash_matches_softmax():
    rng = np.random.default_rng(5)
    T, cap = 40, 64
    q = bits_np(roundbf_np(rng.normal(0, 1, (T, 16, 128)).astype(F)))
    keys = bits_np(roundbf_np(rng.normal(0, 1, (cap, 128)).astype(F)))
    vals = bits_np(roundbf_np(rng.normal(0, 1, (cap, 128)).astype(F)))
    lcb = np.zeros((16, 64), np.uint16)
    mask = np.zeros((T, 1), np.uint32)
    for t in range(T):
        complete = (t + 1) // 4
        if complete:
            chosen = rng.choice(complete, size=min(complete, 3), replace=False)
            for b in chosen:
                mask[t, 0] |= np.uint32(1) << np.uint32(b)
    out = bf_np(xp.flash(q, keys, vals, lcb, lcb, cap, 0, True, mask))
    plain = xp.flash(q, keys, vals, lcb, lcb, cap, 0, True)
    everything = np.full((T, 1), 0xFFFF, np.uint32)
    assert np.array_equal(xp.flash(q, keys, vals, lcb, lcb, cap, 0, True, everything), plain)
    qf, kf, vf = bf_np(q), bf_np(keys), bf_np(vals)
    worst = 0.0
    for t in range(T):
        kp = np.arange(t + 1)
        b = kp // 4
        seen = (b >= (t + 1) // 4) | (((mask[t, 0] >> np.minimum(b, 31).astype(np.uint32)) & 1) == 1)
        for h in (0, 7, 15):
            ref = _softmax_ref(qf[t, h], kf[:t + 1], vf[:t + 1], seen)
            err = float(np.max(np.abs(out[t, h * 128:(h + 1) * 128] - ref)))
            worst = max(worst, err / (float(np.max(np.abs(ref))) + 1e-3))
    print(f"  masked flash vs FP64 softmax: worst relative {worst:.2e}")
    assert worst < 2e-2
    assert not np.array_equal(out, bf_np(plain))


def test_decode_twin_budget(oracle_weights, model_dir):
    # (dense attention equals an all-selected mask: test_masked_flash_matches_softmax here,
    # and the GPU runtime against its dense twin)
    adapters = ad.Adapters(model_dir[0])
    ctx, steps = 32, 14
    covering = exact.ExactDecoder(oracle_weights, ctx, 16, qsa=ad.QsaTwin(adapters, ctx, 32))
    small = exact.ExactDecoder(oracle_weights, ctx, 16, qsa=ad.QsaTwin(adapters, ctx, 8))
    tokens = [1] + [500 + 3 * k for k in range(steps - 1)]
    differs = []
    for pos, tok in enumerate(tokens):
        d = covering.step(tok, pos)[0]
        s = small.step(tok, pos)[0]
        if (pos + 1) // 4 <= 2:  # no query sees more than budget / 4 = 2 complete blocks
            assert np.array_equal(s, d), pos
        else:
            differs.append(not np.array_equal(s, d))
    assert any(differs)
