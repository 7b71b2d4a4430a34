"""The runtime's RoPE tables against the CPU restatement (oracle/rope.py), bit for bit.

The runtime builds the tables on the host (plamo_rope_table, the builder `load_model` uploads)
with the arithmetic of `init_rope` (Kernels.metal:212-219) and the global factors of
`rotated` (Kernels.metal:264-267).  The oracle's closed form is pinned independently by
tests/test_oracle_model.py (phase-0 identity, pair-norm preservation).  Host only: no GPU.
"""
import ctypes

import numpy as np

from oracle import rope
from oracle.bf16 import bits_np
from plamo_hip import native


def runtime_table(freqs, rows, glob):
    lib = native.load()
    f = (ctypes.c_double * 64)(*freqs)
    out = np.zeros(rows * 64, np.uint32)
    err = ctypes.create_string_buffer(256)
    rc = lib.plamo_rope_table(f, rows, 1 if glob else 0, out.ctypes.data, err, 256)
    assert rc == 0, err.value
    t = out.reshape(rows, 64)
    return (t & 0xffff).astype(np.uint16), (t >> 16).astype(np.uint16)


def test_local_table_matches_oracle_bitwise():
    f_local, _ = rope.synthetic_frequencies()
    c, s = runtime_table(f_local, rope.LOCAL_ROWS, False)
    oc, os_ = rope.local_table(f_local, rope.LOCAL_ROWS)
    assert np.array_equal(c, bits_np(oc)) and np.array_equal(s, bits_np(os_))


def test_global_table_matches_oracle_bitwise():
    _, f_full = rope.synthetic_frequencies()
    rows = 4096
    c, s = runtime_table(f_full, rows, True)
    oc, os_ = rope.global_table(f_full, rows)
    assert np.array_equal(c, bits_np(oc)) and np.array_equal(s, bits_np(os_))


def test_rope_table_rejects_bad_arguments():
    lib = native.load()
    f = (ctypes.c_double * 64)(*([1.0] * 64))
    err = ctypes.create_string_buffer(256)
    out = np.zeros(64, np.uint32)
    assert lib.plamo_rope_table(f, 0, 0, out.ctypes.data, err, 256) != 0
    assert lib.plamo_rope_table(f, 40000, 0, out.ctypes.data, err, 256) != 0
