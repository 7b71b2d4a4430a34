"""Pins of the model oracle (oracle/model.py).

Kernel-level functions are pinned by closed forms from the reference's own kernel tests;
the assembled forward is pinned against an independent textbook FP32/FP64 forward with the
reference's acceptance rule (scripts/verify.py:62-63: argmax equal, RMSE < 0.2, cos > 0.999)
plus a tighter bound that a dropped term, wrong offset or transposed operand would break.
"""
import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import rope
from oracle.bf16 import bf_t, bits_t, roundbf_np, roundbf_t


class _Freqs:
    def __init__(self):
        self.f_local, self.f_full = rope.synthetic_frequencies()


def _bf(v):
    return roundbf_np(np.asarray(v, np.float32))


def test_linear_brute_force():
    # PlamoTests.swift:327-364: y = roundbf(W.x) with W [m][n] row-major, tolerance 1e-4
    n, m = 128, 35
    for batch in (1, 3, 16, 33):
        w = _bf((np.arange(n * m) % 17 - 8) / 16).reshape(m, n)
        x = _bf((np.arange(n * batch) % 11 - 5) / 8).reshape(batch, n)
        y = roundbf_t(torch.from_numpy(x) @ torch.from_numpy(w).T).numpy()
        for t in range(batch):
            for r in range(m):
                s = np.float32(0)
                for k in range(n):
                    s = np.float32(s + np.float32(w[r, k] * x[t, k]))
                assert abs(y[t, r] - _bf(s)) <= 1e-4


def test_norm_closed_form_and_offsets():
    # constant rows normalise to +-1 exactly before the gain; gains follow roundbf(bf(w)+offset)
    x = torch.full((2, 1536), 3.0)
    x[1] = -0.5
    zero = torch.zeros(1536, dtype=torch.int32)
    z = om.norm(x, zero, 1.0)
    assert torch.all(z[0] == 1.0) and torch.all(z[1] == -1.0)
    post = bits_t(torch.full((1536,), 0.8))
    post_mlp = bits_t(torch.full((1536,), 0.9105573))
    assert torch.all(om.gain(post, 0.2) == 1.0)
    assert torch.all(om.gain(post_mlp, om.POST_MLP_OFFSET) == 1.0)
    assert torch.all(om.gain(zero, 0.2) == roundbf_t(torch.tensor(0.2)))


def test_rope_identity_at_zero_and_norm_preserving():
    f_local, f_full = rope.synthetic_frequencies()
    lc, ls = rope.local_table(f_local, 64)
    gc, gs = rope.global_table(f_full, 64)
    z = roundbf_t(torch.randn(5, 128))
    out0 = om.rotate(z, torch.from_numpy(lc[0]), torch.from_numpy(ls[0]))
    assert torch.equal(out0, z)
    # textbook complex rotation: (a + ib) * (c + is) per pair (d, d+64)
    p = 37
    for c, s, scale in ((lc, ls, 1.0), (gc, gs, 1.5545177444479562)):
        r = om.rotate(z, torch.from_numpy(c[p]), torch.from_numpy(s[p]))
        ang = p * torch.tensor(f_local if scale == 1.0 else f_full, dtype=torch.float64)
        a, b = z[:, :64].double(), z[:, 64:].double()
        ra = (a * torch.cos(ang) - b * torch.sin(ang)) * scale
        rb = (b * torch.cos(ang) + a * torch.sin(ang)) * scale
        want = torch.cat([ra, rb], 1)
        assert torch.allclose(r.double(), want, atol=0.05, rtol=0.02)


@pytest.mark.parametrize("full", [True, False])
def test_attention_window_mean_with_ring(full):
    # PlamoTests.swift:156-194: zero scores -> mean of V over the visible window, ring wrap
    start = 65 if full else 4090
    base = 0 if full else 2043
    context = start + 2 if full else 8192
    o = om.Oracle.__new__(om.Oracle)
    o.dots = "exact"  # correctly rounded dot products: the same on every machine
    o.w = _Freqs()
    o.context = context
    o.batch_limit = 16
    cap = context if full else 2064
    o.capacity = [cap if om.is_global(i) == full else 2064 for i in range(16)]
    layer = 7 if full else 0
    lc, ls = rope.local_table(o.w.f_local, 2064)
    o.local = (torch.from_numpy(lc), torch.from_numpy(ls))
    o.keys = [torch.zeros(c, 128, dtype=torch.int32) for c in o.capacity]
    o.values = [torch.zeros(c, 128, dtype=torch.int32) for c in o.capacity]
    for pos in range(base, start + 2):
        o.values[layer][pos % cap] = bits_t(torch.full((128,), float(pos % 17 - 8)))
    q = torch.zeros(2, 16, 128)
    out = o._attention(layer, q, 2, start)
    for t in range(2):
        begin = 0 if full else start + t - 2047
        vals = np.array([p % 17 - 8 for p in range(begin, start + t + 1)], np.float64)
        assert torch.allclose(out[t], torch.full((2048,), float(vals.mean())), atol=3e-4)


@pytest.mark.slow
def test_forward_matches_textbook(oracle_weights, golden):
    prompt = golden["config1"]["prompt"]
    o = om.Oracle(oracle_weights, context=96)
    o.prefill(prompt)
    ours = o.logits_fp32.double()
    ref = om.textbook_logits(oracle_weights, prompt).double()
    rmse = float(torch.sqrt(torch.mean((ours - ref) ** 2)))
    cos = float(torch.dot(ours, ref) / (ours.norm() * ref.norm()))
    assert int(ours.argmax()) == int(ref.argmax())
    assert rmse < 0.2 and cos > 0.999       # the reference's acceptance rule
    assert rmse < 0.05 and cos > 0.9995     # tight enough to catch a dropped term or wrong offset
