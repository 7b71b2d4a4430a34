"""The allocation-free decode attention entry point (plamo_kernel_attention_decode_static)
against the allocating one it varies (plamo_kernel_attention_decode), through the C ABI.

Both run the same kernels, so outputs and cache writes must be bit-identical: two calls in
a row, the second smaller than the first (the shared static scratch keeps the first call's
contents), local and global layers, the in-kernel ticket merge (> 1 partition) and the
one-partition path.  Calls beyond the static scratch (more than 8192 visible keys) fail
with a clear error before any device work.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import rope
from oracle.bf16 import bits_np
from plamo_hip import native

pytestmark = pytest.mark.gpu


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _tables(rows_global):
    f_local, f_full = rope.synthetic_frequencies()
    out = []
    for freqs, rows, glob in ((f_local, rope.LOCAL_ROWS, 0), (f_full, rows_global, 1)):
        t = np.zeros(rows * 64, np.uint32)
        err = ctypes.create_string_buffer(256)
        assert native.load().plamo_rope_table((ctypes.c_double * 64)(*freqs), rows, glob, t.ctypes.data, err,
                                              256) == 0
        out.append(_dev(t.view(np.int32)))
    return out


def _call(static, rows, cap, positions, full, seed, lrope, grope):
    """One call on fresh inputs from `seed` -> (output bits, keys, values after the call)."""
    lib = native.load()
    rng = np.random.default_rng(seed)
    qkv = _dev((bits_np(rng.standard_normal((rows, 2304)).astype(np.float32)).astype(np.uint32) << 16)
               .view(np.float32))
    keys = _dev(bits_np(rng.standard_normal((rows, cap, 128)).astype(np.float32)).view(np.int16))
    values = _dev(bits_np(rng.standard_normal((rows, cap, 128)).astype(np.float32)).view(np.int16))
    qn = _dev(bits_np((rng.standard_normal(128) * 0.1).astype(np.float32)).view(np.int16))
    kn = _dev(bits_np((rng.standard_normal(128) * 0.1).astype(np.float32)).view(np.int16))
    out = torch.full((rows, 2048), -1, dtype=torch.int16, device="cuda")
    pos = (ctypes.c_int32 * rows)(*positions)
    args = (qkv.data_ptr(), qn.data_ptr(), kn.data_ptr(), keys.data_ptr(), values.data_ptr(), cap, pos, rows,
            1 if full else 0, lrope.data_ptr(), grope.data_ptr(), out.data_ptr(), 0)
    if static:
        err = ctypes.create_string_buffer(256)
        rc = lib.plamo_kernel_attention_decode_static(*args, err, 256)
        assert rc == 0, err.value
    else:
        assert lib.plamo_kernel_attention_decode(*args) == 0
    torch.cuda.synchronize()
    return out.cpu().numpy(), keys.cpu().numpy(), values.cpu().numpy()


@pytest.mark.parametrize("full,first,second", [
    # (rows, cap, positions) of two calls in a row, the second smaller
    (True, (4, 8192, [8188, 8189, 8190, 8191]), (2, 300, [10, 299])),
    (False, (3, 2064, [4090, 4091, 4092]), (1, 2064, [40])),
])
def test_static_entry_matches_allocating_entry(full, first, second):
    lrope, grope = _tables(8192)
    for k, (rows, cap, positions) in enumerate((first, second)):
        print(f"  no-alloc call {k}: full={full} rows={rows} cap={cap} positions={positions}", flush=True)
        a = _call(False, rows, cap, positions, full, 100 + k, lrope, grope)
        b = _call(True, rows, cap, positions, full, 100 + k, lrope, grope)
        for x, y in zip(a, b):
            assert np.array_equal(x, y)
        assert not np.all(a[0] == -1)   # the outputs were written


def test_static_entry_rejects_calls_beyond_its_scratch():
    lib = native.load()
    err = ctypes.create_string_buffer(256)
    pos = (ctypes.c_int32 * 1)(8192)   # 8193 visible keys: 129 partitions
    rc = lib.plamo_kernel_attention_decode_static(1, 1, 1, 1, 1, 9000, pos, 1, 1, 1, 1, 1, 0, err, 256)
    assert rc == 1 and b"static scratch" in err.value
