"""Prefill attention (MFMA flash kernel) against an FP32 reference, through the C ABI.

The reference's prefill attention (Runtime.swift:389-444) takes BF16 queries and keys,
FP32 scores scaled by 1/sqrt(128) before the max, an FP32 softmax over the visible keys
(the 2048-key window on local layers, all earlier keys on global layers) and
roundbf(sum p v).  Local keys are rotated with coordinate key_pos - base of the query's
16-token chunk (base = max(0, chunk_start - 2047), chunks counted from p0), with the BF16
rounding of `rotate` (Runtime.swift:277-285).

The kernel accumulates on MFMA with P split into two BF16 halves (P keeps ~16 significant
bits), so its sums differ from FP32 in the last bits: every output must be within one BF16
ulp of the reference plus an absolute 2^-14 (outputs that cancel to near zero carry the
absolute error of sums whose terms are O(1)), and at most 1 % of the outputs may differ
at all.
"""
import numpy as np
import pytest
import torch

from oracle import rope
from oracle.bf16 import bf_np, bits_np, roundbf_np
from plamo_hip import native

pytestmark = pytest.mark.gpu

SCALE = np.float32(0.08838834764831845)
WINDOW = 2048


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def local_rope_table():
    freqs = (10000.0 ** (-np.arange(64, dtype=np.float64) / 64)).astype(np.float32)
    c, s = rope.local_table(freqs, rope.LOCAL_ROWS)
    packed = bits_np(c).astype(np.uint32) | (bits_np(s).astype(np.uint32) << 16)
    return c, s, packed


def rotate(k, c, s):
    a, b = k[..., :64], k[..., 64:]
    ra = roundbf_np(roundbf_np(a * c) + roundbf_np(-b * s))
    rb = roundbf_np(roundbf_np(b * c) + roundbf_np(a * s))
    return np.concatenate([ra, rb], -1)


def reference(q, keys, values, cap, p0, full, c, s):
    """q [T][16][128] FP32 (BF16 values); keys/values [cap][128] FP32 (BF16 values)."""
    T = q.shape[0]
    out = np.zeros((T, 16, 128), np.float32)
    for t in range(T):
        pos = p0 + t
        first = 0 if full else max(0, pos - (WINDOW - 1))
        kp = np.arange(first, pos + 1)
        k = keys[kp % cap]
        if not full:
            chunk = p0 + (t // 16) * 16
            base = max(0, chunk - (WINDOW - 1))
            k = rotate(k, c[kp - base], s[kp - base])
        v = values[kp % cap]
        qt = torch.from_numpy(q[t])
        sc = (qt @ torch.from_numpy(k).T) * torch.tensor(SCALE)
        m = sc.max(-1, keepdim=True).values
        e = torch.exp(sc - m)
        p = e / e.sum(-1, keepdim=True)
        out[t] = (p @ torch.from_numpy(v)).numpy()
    return roundbf_np(out)


def ulp(x):
    a = np.maximum(np.abs(x), np.float32(1e-30))
    return np.exp2(np.floor(np.log2(a)) - 7).astype(np.float32)


@pytest.fixture(scope="module")
def lib():
    return native.load()


@pytest.mark.parametrize("p0,tokens,cap,full", [
    (0, 100, 2064, False),     # ragged token count, keys from position 0
    (2040, 24, 2080, False),   # chunk bases 0 and 9 in one call
    (3000, 40, 2112, False),   # chunk-relative coordinates and a wrapped ring
    (0, 64, 64, True),         # global, keys exactly the tokens
    (500, 37, 600, True),      # global, long prefix: key tiles split over two workgroups
    (1100, 50, 1200, True),    # global, three parts merged
])
def test_flash_prefill_matches_fp32(lib, p0, tokens, cap, full):
    print(f"  flash p0={p0} tokens={tokens} cap={cap} full={full}", flush=True)
    rng = np.random.default_rng(p0 + tokens)
    q = roundbf_np(rng.standard_normal((tokens, 16, 128)).astype(np.float32))
    keys = roundbf_np(rng.standard_normal((cap, 128)).astype(np.float32))
    values = roundbf_np(rng.standard_normal((cap, 128)).astype(np.float32))
    c, s, packed = local_rope_table()
    want = reference(q, keys, values, cap, p0, full, c, s).reshape(tokens, 2048)
    qd = dev(bits_np(q).view(np.int16))
    kd = dev(bits_np(keys).view(np.int16))
    vd = dev(bits_np(values).view(np.int16))
    rd = dev(packed.view(np.int32))
    out = torch.full((tokens, 2048), -1, dtype=torch.int16, device="cuda")
    rc = lib.plamo_kernel_attention_prefill(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), cap, p0, tokens,
                                            1 if full else 0, rd.data_ptr(), out.data_ptr(), 0)
    assert rc == 0
    torch.cuda.synchronize()
    got = bf_np(out.cpu().numpy().view(np.uint16))
    diff = np.abs(got - want)
    over = diff > ulp(want) * 1.001 + 2.0 ** -14
    w = np.unravel_index(np.argmax(diff / ulp(want)), diff.shape)
    print(f"    mismatched {np.mean(diff > 0):.4f}, over 1 ulp {int(over.sum())}, worst {want[w]} vs {got[w]}"
          f" at {w}, max abs {diff.max()}", flush=True)
    assert not over.any()
    assert np.mean(diff > 0) < 0.01, float(np.mean(diff > 0))


def test_flash_prefill_rejects_short_cache(lib):
    # a local call whose visible keys do not fit the ring is refused before any launch
    rc = lib.plamo_kernel_attention_prefill(1, 1, 1, 100, 200, 16, 0, 1, 1, 0)
    assert rc != 0
