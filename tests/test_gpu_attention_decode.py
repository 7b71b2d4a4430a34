"""Decode attention kernel (plamo_kernel_attention_decode) against the reference's own
attention checks, restated for the HIP kernel and computed independently of the GPU.

* Window mean with ring wrap (Tests/PlamoTests/PlamoTests.swift:156-194): with zero queries
  every visible key scores 0, so the output of every dimension is the mean of the visible
  values.  Local rows at positions 4090 and 4091 (window base 2043, 2064-slot ring, so the
  window wraps the ring) and global rows at 65 and 66; value of position p is p % 17 - 8;
  accuracy 3e-4 as in the reference.
* Partitioned vs dense (Tests/PlamoTests/AttentionTests.swift:6-75): the reference checks its
  split `attention` + `attention_merge` against `matrix` + `softmax` + `attend` within 2e-3 on
  patterned keys, values and queries for counts 19 .. 32,768 (global rows at count - batch ..
  count - 1; local rows at 4090.. with a 2064-slot ring; 2050 is the base > 0 case).  Here the
  dense side is an FP32 torch restatement of the same layer (q/k RMSNorm, RoPE, the new key
  and value at pos % capacity, softmax over the visible keys, P.V), and the kernel's BF16
  output must be within 2e-3 of its unrounded FP32 result.  The 32,768-key rows have 512
  partitions, merged by attn_merge_kernel; the 4096/8192-key rows go through the in-kernel
  ticket merge.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import rope
from oracle.bf16 import bf_np, bits_np, bf_t, roundbf_t
from plamo_hip import native

pytestmark = pytest.mark.gpu

SCALE = np.float32(0.08838834764831845)
WINDOW = 2048


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def rope_packed(freqs, rows, glob):
    lib = native.load()
    out = np.zeros(rows * 64, np.uint32)
    err = ctypes.create_string_buffer(256)
    assert lib.plamo_rope_table((ctypes.c_double * 64)(*freqs), rows, 1 if glob else 0, out.ctypes.data, err,
                                256) == 0, err.value
    return out


def pattern(n, mul, mod, off):
    """(i * mul) % mod - off, over 32, as BF16 bits (AttentionTests.swift:20-22)."""
    i = np.arange(n, dtype=np.int64)
    return bits_np(((i * mul) % mod - off).astype(np.float32) / np.float32(32))


def run_kernel(qkv, qn, kn, keys, values, cap, positions, full, lrope, grope):
    """qkv FP32 [rows][2304]; keys/values uint16 [rows][cap][128] -> (output bits, cache after)."""
    lib = native.load()
    rows = len(positions)
    qd = dev(qkv.astype(np.float32))
    kd = dev(keys.view(np.int16))
    vd = dev(values.view(np.int16))
    qnd, knd = dev(qn.view(np.int16)), dev(kn.view(np.int16))
    ld = dev(lrope.view(np.int32))
    gd = dev(grope.view(np.int32)) if grope is not None else ld
    out = torch.full((rows, 2048), -1, dtype=torch.int16, device="cuda")
    pos = (ctypes.c_int32 * rows)(*positions)
    rc = lib.plamo_kernel_attention_decode(qd.data_ptr(), qnd.data_ptr(), knd.data_ptr(), kd.data_ptr(),
                                           vd.data_ptr(), cap, pos, rows, 1 if full else 0, ld.data_ptr(),
                                           gd.data_ptr(), out.data_ptr(), 0)
    assert rc == 0
    torch.cuda.synchronize()
    return (out.cpu().numpy().view(np.uint16), kd.cpu().numpy().view(np.uint16),
            vd.cpu().numpy().view(np.uint16))


def reference(qkv, qn, kn, keys, values, cap, pos, full, tables):
    """FP32 restatement of one row (Runtime.swift:389-444 for a one-token chunk): returns the
    unrounded attention output [2048] and the new key and value bits."""
    lc, ls, gc, gs = tables
    x = torch.from_numpy(qkv.astype(np.float32))
    qn_t = torch.from_numpy(qn.astype(np.int32))
    kn_t = torch.from_numpy(kn.astype(np.int32))
    zq = om.norm(x[:2048].reshape(16, 128), qn_t, 1.0)
    zk = om.norm(x[2048:2176].reshape(1, 128), kn_t, 1.0)[0]
    first = 0 if full else max(0, pos - (WINDOW - 1))
    if full:
        q = om.rotate(zq, gc[pos], gs[pos])
        knew = om.rotate(zk, gc[pos], gs[pos])
    else:
        q = om.rotate(zq, lc[pos - first], ls[pos - first])
        knew = zk
    vnew = x[2176:2304]
    kb = bf_t(torch.from_numpy(keys.astype(np.int32)))
    vb = bf_t(torch.from_numpy(values.astype(np.int32)))
    kb[pos % cap] = roundbf_t(knew)
    vb[pos % cap] = roundbf_t(vnew)
    kp = torch.arange(first, pos + 1)
    k = kb[kp % cap]
    if not full:
        k = om.rotate(k, lc[kp - first], ls[kp - first])
    v = vb[kp % cap]
    sc = (q @ k.T) * torch.tensor(SCALE)
    m = sc.max(-1, keepdim=True).values
    e = torch.exp(sc - m)
    p = e / e.sum(-1, keepdim=True)
    return (p @ v).reshape(2048).numpy(), roundbf_t(knew).numpy(), roundbf_t(vnew).numpy()


@pytest.fixture(scope="module")
def tables():
    f_local, f_full = rope.synthetic_frequencies()
    lc, ls = rope.local_table(f_local, rope.LOCAL_ROWS)
    gc, gs = rope.global_table(f_full, 32768)
    t = tuple(torch.from_numpy(a) for a in (lc, ls, gc, gs))
    return t, rope_packed(f_local, rope.LOCAL_ROWS, False), rope_packed(f_full, 32768, True)


@pytest.mark.parametrize("full", [False, True])
def test_window_mean_with_ring_wrap(tables, full):
    # PlamoTests.swift:156-194: zero scores -> the mean of the visible values
    _, lrope, grope = tables
    start, base = (65, 0) if full else (4090, 2043)
    cap = start + 2 - base if full else 2064
    positions = [start, start + 1]
    print(f"  window mean full={full} positions={positions} cap={cap}", flush=True)
    values = np.zeros((2, cap, 128), np.uint16)
    for p in range(base, start + 2):
        values[:, p % cap, :] = bits_np(np.float32(p % 17 - 8))
    rng = np.random.default_rng(7)
    keys = bits_np(rng.standard_normal((2, cap, 128)).astype(np.float32))
    qkv = np.zeros((2, 2304), np.float32)
    qkv[:, 2048:2176] = bf_np(bits_np(rng.standard_normal((2, 128)).astype(np.float32)))
    for r, p in enumerate(positions):
        qkv[r, 2176:] = np.float32(p % 17 - 8)
    qn = kn = np.zeros(128, np.uint16)
    out, kc, vc = run_kernel(qkv, qn, kn, keys, values, cap, positions, full, lrope, grope)
    for r, p in enumerate(positions):
        begin = 0 if full else p - 2047
        want = np.float32(sum(k % 17 - 8 for k in range(begin, p + 1)) / (p - begin + 1))
        got = bf_np(out[r])
        assert np.all(np.abs(got - want) <= 3e-4), (p, float(want), float(got[0]))
        assert np.all(vc[r, p % cap] == bits_np(np.float32(p % 17 - 8)))


CASES = [  # (count, rows, full): AttentionTests.swift:16 with batches capped at four rows
    (19, 3, True), (513, 4, True), (131, 3, True), (4096, 4, True), (8192, 4, True), (32768, 1, True),
    (32768, 4, True), (2048, 3, False), (2050, 3, False), (19, 3, False)]
# local rows: count 2048 -> positions 2045..2047 (windows from key 0, base 0); count 2050 ->
# positions 4090.. (window base 2043.., the ring wrapped); count 19 -> positions 16..18


@pytest.mark.parametrize("count,rows,full", CASES)
def test_partitioned_matches_dense_fp32(tables, count, rows, full):
    (lc, ls, gc, gs), lrope, grope = tables
    if full:
        cap, positions = count, [count - rows + r for r in range(rows)]
    elif count > WINDOW:
        cap, positions = 2064, [4090 + r for r in range(rows)]
    else:
        cap, positions = 2064, [count - rows + r for r in range(rows)]
    print(f"  partitioned count={count} rows={rows} full={full} cap={cap} positions={positions}", flush=True)
    keys = np.broadcast_to(pattern(cap * 128, 17, 43, 21).reshape(cap, 128), (rows, cap, 128)).copy()
    values = np.broadcast_to(pattern(cap * 128, 13, 41, 20).reshape(cap, 128), (rows, cap, 128)).copy()
    qkv = np.zeros((rows, 2304), np.float32)
    qkv[:, :2048] = bf_np(pattern(rows * 2048, 7, 47, 23)).reshape(rows, 2048)
    kv_new = bf_np(pattern(rows * 256, 11, 37, 18)).reshape(rows, 256)
    qkv[:, 2048:] = kv_new
    rng = np.random.default_rng(count + rows)
    qn = bits_np((rng.standard_normal(128) * 0.1).astype(np.float32))
    kn = bits_np((rng.standard_normal(128) * 0.1).astype(np.float32))
    out, kc, vc = run_kernel(qkv, qn, kn, keys, values, cap, positions, full, lrope, grope if full else None)
    worst = 0.0
    for r, p in enumerate(positions):
        want, knew, vnew = reference(qkv[r], qn, kn, keys[r], values[r], cap, p, full, (lc, ls, gc, gs))
        got = bf_np(out[r])
        assert np.all(np.isfinite(got))
        err = float(np.max(np.abs(got.astype(np.float64) - want.astype(np.float64))))
        worst = max(worst, err)
        assert err <= 2e-3, (count, rows, full, p, err)
        # the new key and value landed in the row's slice at pos % capacity
        assert np.array_equal(kc[r, p % cap], bits_np(knew)) and np.array_equal(vc[r, p % cap], bits_np(vnew))
    print(f"    max abs error {worst:.2e}", flush=True)

