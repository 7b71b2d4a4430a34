"""Trained adapters on the CPU: the auxiliary.safetensors checks of Auxiliary.swift:14-62
(through the native library, no device), and the MTP draft restatement
(oracle/adapters.py) pinned against the same formula in FP64."""
import json
import os
import struct

import numpy as np
import pytest

from oracle import adapters as ad, exact
from oracle.bf16 import bf_np, bits_np
from plamo_hip import native, synth

F = np.float32


@pytest.fixture(scope="module")
def model(model_dir):
    return model_dir


def _rewrite(src, dst, edit_header=None, edit_bytes=None):
    raw = open(src, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    body = raw[8 + n:]
    if edit_header:
        edit_header(header)
    blob = json.dumps(header, separators=(",", ":")).encode()
    blob += b" " * ((-(8 + len(blob))) % 64)
    out = struct.pack("<Q", len(blob)) + blob + body
    if edit_bytes:
        out = edit_bytes(out)
    with open(dst, "wb") as f:
        f.write(out)


def test_adapter_file_checks(model, tmp_path):
    d, sha = model
    src = os.path.join(d, "auxiliary.safetensors")
    native.check_aux(src, sha)
    with pytest.raises(native.PlamoError, match="Incompatible trained adapters"):
        native.check_aux(src)  # trained against another teacher: the pinned checksum differs
    with pytest.raises(native.PlamoError, match="Trained adapters missing; run scripts/train_auxiliary.py --collect"):
        native.check_aux(str(tmp_path / "missing.safetensors"), sha)
    bad = str(tmp_path / "aux.safetensors")
    cases = [
        (None, lambda b: b[:8], "Invalid adapter size"),
        (None, lambda b: struct.pack("<Q", 2 ** 21) + b[8:], "Invalid adapter header"),
        (None, lambda b: struct.pack("<Q", struct.unpack("<Q", b[:8])[0] + 3) + b[8:], "Invalid adapter header"),
        (lambda h: h["__metadata__"].update(format="plamo-aux-v0"), None, "Incompatible trained adapters"),
        (lambda h: h["__metadata__"].update(rank="128"), None, "Incompatible trained adapters"),
        (lambda h: h["__metadata__"].update(qsa_steps="0"), None, "Incompatible trained adapters"),
        (lambda h: h["__metadata__"].update(mtp_steps="x"), None, "Incompatible trained adapters"),
        (lambda h: h["__metadata__"].pop("teacher_sha256"), None, "Incompatible trained adapters"),
        (lambda h: h["mtp.heads.0.up.weight"].update(dtype="F16"), None, "Invalid adapter tensor: mtp.heads.0.up.weight"),
        (lambda h: h["mtp.heads.0.down.weight"].update(shape=[256, 1536]), None,
         "Invalid adapter tensor: mtp.heads.0.down.weight"),
        (lambda h: h["qsa.15.proj.weight"]["data_offsets"].__setitem__(0, h["qsa.15.proj.weight"]["data_offsets"][0] + 2),
         None, "Invalid adapter tensor: qsa.15.proj.weight"),
        (lambda h: h.pop("qsa.7.k_norm.weight"), None, "Invalid adapter tensor: qsa.7.k_norm.weight"),
    ]
    for edit_h, edit_b, msg in cases:
        _rewrite(src, bad, edit_h, edit_b)
        with pytest.raises(native.PlamoError, match=msg):
            native.check_aux(bad, sha)
    # the QSA tensors are only read when the indexers are used (Runtime.swift:248)
    _rewrite(src, bad, lambda h: h.pop("qsa.7.k_norm.weight"))
    native.check_aux(bad, sha, mtp=True, qsa=False)


def test_mtp_down_order_and_bound():
    rng = np.random.default_rng(3)
    w = bits_np((rng.standard_normal((64, 256)) * 0.02).astype(F))
    a = bf_np(bits_np(rng.standard_normal(256).astype(F)))
    got = ad.mtp_down(w, a).astype(np.float64)
    want = bf_np(w).astype(np.float64) @ a.astype(np.float64)
    bound = 4 * 2.0 ** -23 * (np.abs(bf_np(w)).astype(np.float64) @ np.abs(a).astype(np.float64))
    assert np.all(np.abs(got - want) <= bound)
    # integer-valued operands: every partial sum is exact
    wi = bits_np(rng.integers(-60, 61, (64, 256)).astype(F))
    ai = rng.integers(-60, 61, 256).astype(F)
    assert np.array_equal(ad.mtp_down(wi, ai).astype(np.float64), bf_np(wi).astype(np.float64) @ ai.astype(np.float64))
    # a transposed column pairing is not the kernel's order: different bits somewhere
    swapped = ad.mtp_down(w.reshape(64, 64, 4)[:, :, [2, 3, 0, 1]].reshape(64, 256), a)
    assert not np.array_equal(swapped, ad.mtp_down(w, a))


def test_mtp_draft_tracks_textbook(model, oracle_weights):
    d, _ = model
    adp = ad.Adapters(d)
    ex = exact.ExactDecoder(oracle_weights, 16, 16)
    rng = np.random.default_rng(4)
    for first in (500, 12345, 107000):
        hidden = bf_np(bits_np(rng.standard_normal(1536).astype(F)))
        bits, tok = ad.mtp_draft(ex, adp, hidden, first)
        ref = ad.textbook_draft(oracle_weights.embed_bits, ex.head, adp, hidden, first)
        got = bf_np(bits).astype(np.float64)
        err = np.abs(got - ref)
        # BF16 logits of the same z: within one BF16 ulp plus what 1-ulp differences in the
        # BF16 intermediates move (measured max well below)
        assert np.sqrt(np.mean(err ** 2)) < 5e-3 and err.max() < 0.05, (first, err.max())
        assert ref.max() - ref[tok] <= max(2.0 ** (np.floor(np.log2(abs(ref.max()))) - 6), 0.02), first
