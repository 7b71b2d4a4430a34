"""RoPE cos/sin tables (test infrastructure only).

Reference arithmetic:
* local table, ``init_rope`` (Kernels.metal:212-219): ``phase = float(pos) * f_local[d]`` in
  FP32, stored as ``(bits(cos(phase)), bits(sin(phase)))``; rows = ``min(context, 2064)``
  (Runtime.swift:266).
* global factors, ``rotated`` with ``full`` (Kernels.metal:264-267):
  ``angle = float(pos) * f_full[d]``; ``c = roundbf(roundbf(cos(angle)) * 1.5545177444479562f)``
  and likewise ``s``.

Metal's ``cos``/``sin`` cannot be reproduced here, so both the runtime and this oracle
evaluate cos/sin of the (exact) FP32 angle in double precision with the C library
(``math.cos`` is glibc's ``cos``, the same routine the runtime's C++ table builder calls),
round to FP32, then apply the BF16 roundings above.  Runtime and oracle tables are compared
bit for bit in tests/test_rope.py (through plamo_rope_table, the runtime's host builder); the closed
form is pinned in tests/test_oracle_model.py by the textbook rotary
identity (rotation preserves the pair norm to BF16 accuracy, phase 0 is the identity).
"""
import math

import numpy as np

from .bf16 import bits_np, bf_np, roundbf_np

MSCALE = np.float32(1.5545177444479562)
LOCAL_ROWS = 2064


def _cos_sin(angles):
    flat = angles.reshape(-1).astype(np.float64)
    c = np.fromiter((math.cos(a) for a in flat.tolist()), dtype=np.float64, count=flat.size)
    s = np.fromiter((math.sin(a) for a in flat.tolist()), dtype=np.float64, count=flat.size)
    return c.astype(np.float32).reshape(angles.shape), s.astype(np.float32).reshape(angles.shape)


def angles(rows, freqs):
    pos = np.arange(rows, dtype=np.float32)[:, None]
    return (pos * np.asarray(freqs, dtype=np.float32)[None, :]).astype(np.float32)


def local_table(freqs, rows):
    """-> (cos, sin) FP32 [rows, 64] holding BF16 values (init_rope)."""
    c, s = _cos_sin(angles(rows, freqs))
    return bf_np(bits_np(c)), bf_np(bits_np(s))


def global_table(freqs, rows):
    """-> (cos, sin) FP32 [rows, 64]: roundbf(roundbf(cos) * mscale) (rotated, full)."""
    c, s = _cos_sin(angles(rows, freqs))
    return (roundbf_np((roundbf_np(c) * MSCALE).astype(np.float32)),
            roundbf_np((roundbf_np(s) * MSCALE).astype(np.float32)))


def synthetic_frequencies():
    """The synthetic inverse frequencies used for random-init models, following the
    reference's own test construction ``1/(theta**(arange(64)/64))``
    (scripts/test_auxiliary.py:36) with rope_local_theta 1e4 and rope_theta 1e6
    (Runtime.swift:187)."""
    i = np.arange(64, dtype=np.float64)
    return (1.0 / (10000.0 ** (i / 64.0))).tolist(), (1.0 / (1000000.0 ** (i / 64.0))).tolist()
