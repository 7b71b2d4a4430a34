"""Kernel-level parity on the GPU through the C-ABI kernel entry points.

Known answers from the reference's kernel tests (PackedDecodeTests, ArgmaxTests,
SamplerTests, PlamoTests.testMetalLinearAndMatrix) plus packed == plain bit equality
(PackedTests.swift:6-46: one- and multi-row products of .p12 and raw weights) and
FP32 references for the GEMV/GEMM.  Device memory comes from torch (plumbing only).
"""
import numpy as np
import pytest
import torch

from oracle import exact, p12, sampler
from oracle.bf16 import bf_np, bits_np, roundbf_np
from plamo_hip import native

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def ptr(t):
    return t.data_ptr()


@pytest.fixture(scope="module")
def lib():
    return native.load()


def test_unpack_known_answers(lib):
    payload, table, expected = p12.decode_kat()
    out = torch.empty(expected.size, dtype=torch.int16, device="cuda")
    pd, td = dev(payload), dev(table.view(np.int32))
    assert lib.plamo_kernel_unpack(ptr(pd), ptr(td), ptr(out), expected.size, 0) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16).astype(np.uint32) << 16
    assert np.array_equal(got, expected)


def test_argmax_patterns(lib):
    for count in [1, 31, 32, 33, 255, 256, 257, 1023, 1024, 1025, 107520]:
        for batch in (1, 2, 3):
            for pattern in range(5):
                v = ((np.arange(count * batch) * 17) % 4093 - 2046).astype(np.float32) / 32
                v = v.reshape(batch, count)
                for r in range(batch):
                    if pattern == 1:
                        v[r] = -np.inf
                    elif pattern == 2:
                        v[r] = np.nan
                    elif pattern == 3:
                        v[r] = np.where(np.arange(count) % 2 == 0, np.float32(-0.0), np.float32(0.0))
                    elif pattern == 4:
                        v[r, 0] = np.nan
                        if count > 1:
                            v[r, count - 1] = np.inf
                        if count > 257:
                            v[r, 257] = np.inf
                for compact in (False, True):
                    tested = bf_np(bits_np(v)) if compact else v
                    want = [sampler.argmax_sequential(tested[r]) for r in range(batch)]
                    x = dev(bits_np(v).view(np.int16)) if compact else dev(v)
                    out = torch.empty(batch, dtype=torch.int32, device="cuda")
                    assert lib.plamo_kernel_argmax(ptr(x), ptr(out), count, batch, int(compact), 0) == 0
                    torch.cuda.synchronize()
                    got = (out.cpu().numpy().view(np.uint32)).tolist()
                    assert got == want, (count, batch, pattern, compact)


@pytest.mark.parametrize("logits,history,penalty,ngram,frequency,want", [
    ([1, 2, 2, 0], [], 1, 0, 0, 1),
    ([1, 5, 4], [1], 2, 0, 0, 2),
    ([-1, -5, -4], [1], 2, 0, 0, 0),
    ([0, 5, 4], [1], 1, 0, 0.5, 1),
    ([0, 5, 4], [1, 1, 1], 1, 0, 0.5, 2),
    ([0, 0, 0, 0, 0, 9], [0, 2, 3, 5, 2, 3], 1, 3, 0, 0),
])
def test_select_known_answers(lib, logits, history, penalty, ngram, frequency, want):
    # SamplerTests.swift:5-32 on the GPU
    x = dev(np.array(logits, np.float32))
    h = dev(np.array(history or [0], np.int32))
    out = torch.empty(1, dtype=torch.int32, device="cuda")
    assert lib.plamo_kernel_select(ptr(x), len(logits), ptr(h), len(history), penalty, ngram, frequency, 0.0,
                                   ptr(out), 0) == 0
    torch.cuda.synchronize()
    assert int(out.item()) == want


def test_select_matches_oracle_on_vocab(lib):
    rng = np.random.default_rng(11)
    logits = bf_np(bits_np(rng.standard_normal(107520).astype(np.float32)))
    hist = rng.integers(0, 200, 300).astype(np.int32)
    for penalty, ngram, freq, pres in ((1.1, 4, 0.2, 0.0), (1.3, 2, 0.0, 0.5), (1.0, 3, 0.7, 0.0)):
        want = sampler.select(logits.copy(), hist.tolist(), penalty, ngram, freq, pres)
        x, h = dev(logits.copy()), dev(hist)
        out = torch.empty(1, dtype=torch.int32, device="cuda")
        assert lib.plamo_kernel_select(ptr(x), 107520, ptr(h), len(hist), penalty, ngram, freq, pres, ptr(out), 0) == 0
        torch.cuda.synchronize()
        assert int(out.item()) == want


def _linear(lib, w_bits, x, rows, mode=0, table=None, payload=None):
    m, n = w_bits.shape
    if table is None:
        wd, td = dev(w_bits.view(np.int16)), None
    else:
        wd, td = dev(payload), dev(table.view(np.int32))
    xd = dev(x.astype(np.float32))
    y = torch.empty(rows * m, dtype=torch.int16 if mode == 2 else torch.float32, device="cuda")
    rc = lib.plamo_kernel_linear(ptr(wd), ptr(td) if td is not None else 0, ptr(xd), ptr(y), n, m, rows, mode, 0)
    assert rc == 0
    torch.cuda.synchronize()
    out = y.cpu().numpy()
    return out.view(np.uint16).reshape(rows, m) if mode == 2 else out.reshape(rows, m)


def test_linear_brute_force(lib):
    # PlamoTests.swift:327-364 pattern, widened to the kernel's n = 1536
    n, m = 1536, 36
    w = bits_np((np.arange(n * m) % 17 - 8).astype(np.float32) / 16).reshape(m, n)
    for rows in (1, 2, 3, 4):
        x = roundbf_np((np.arange(n * rows) % 11 - 5).astype(np.float32) / 8).reshape(rows, n)
        y = _linear(lib, w, x, rows)
        ref = (x.astype(np.float64) @ bf_np(w).astype(np.float64).T)
        assert np.all(np.abs(y - roundbf_np(ref.astype(np.float32))) <= 1e-4)


SHAPES = {"qkv": (2304, 1536), "o": (1536, 2048), "gate_up": (12288, 1536), "down": (1536, 6144),
          "head": (107520, 1536)}


@pytest.mark.parametrize("name", list(SHAPES))
def test_linear_packed_equals_plain_and_fp32(lib, name):
    m, n = SHAPES[name]
    rng = np.random.default_rng(7)
    w = bits_np(rng.standard_normal((m, n)).astype(np.float32) * 0.02)
    w[1, :128] = bits_np(np.full(128, 1e-30, np.float32))  # exponent below 108 -> a raw block
    data, offsets, minima = p12.pack(w)
    table = p12.tag(offsets, minima)
    assert (minima == 0).any()
    for rows in (1, 4):
        x = roundbf_np(rng.standard_normal((rows, n)).astype(np.float32))
        mode = 2 if name == "head" else 0
        plain = _linear(lib, w, x, rows, mode)
        packed = _linear(lib, w, x, rows, mode, table=table, payload=data)
        assert np.array_equal(plain.view(np.uint32) if mode == 0 else plain,
                              packed.view(np.uint32) if mode == 0 else packed)
        ref = torch.from_numpy(x) @ torch.from_numpy(bf_np(w)).T
        got = plain if mode == 0 else bf_np(plain)
        ulp = np.abs(roundbf_np(ref.numpy()) - ref.numpy()) * 2 + 1e-6
        err = np.abs(got - ref.numpy())
        # within one BF16 ulp of the FP32 reference
        assert np.all(err <= np.maximum(ulp, np.abs(ref.numpy()) * 2 ** -7) + 1e-6)
        # rows are independent: row r of a 4-row call equals a 1-row call
        if rows == 4:
            single = _linear(lib, w, x[2:3], 1, mode)
            assert np.array_equal(single.view(np.uint32) if mode == 0 else single,
                                  (plain[2:3].view(np.uint32) if mode == 0 else plain[2:3]))


@pytest.mark.parametrize("name", list(SHAPES))
def test_linear_raw_sums_equal_the_twin(lib, name):
    # mode 1 returns the FP32 sums before any rounding: every bit of every lane chain
    # (v_dot2_f32_bf16 steps) and of the butterfly, against csrc/exact_gemv.c, plain and
    # .p12, one and four rows
    m, n = SHAPES[name]
    rng = np.random.default_rng(11)
    w = bits_np(rng.standard_normal((m, n)).astype(np.float32) * 0.02)
    w[3, 128:256] = bits_np(np.full(128, 1e-30, np.float32))  # a raw .p12 block
    data, offsets, minima = p12.pack(w)
    table = p12.tag(offsets, minima)
    wf = bf_np(w)
    x = roundbf_np(rng.standard_normal((4, n)).astype(np.float32))
    x[1, ::7] = roundbf_np(x[1, ::7] * 40)  # outliers (activations are BF16 values)
    want = np.stack([exact.gemv(wf, x[r]) for r in range(4)])
    for rows in (1, 4):
        for packed in (False, True):
            got = _linear(lib, w, x[:rows], rows, 1, table=table if packed else None, payload=data if packed else None)
            bad = int(np.sum(got.view(np.uint32) != want[:rows].view(np.uint32)))
            assert bad == 0, (name, rows, packed, bad)


@pytest.mark.parametrize("m,n,tokens", [(2304, 1536, 130), (1536, 2048, 64), (1536, 6144, 257), (64, 1536, 17),
                                          (2304, 1536, 2048), (200, 512, 300)])
def test_gemm_matches_fp32_and_packed(lib, m, n, tokens):
    rng = np.random.default_rng(m + tokens)
    w = bits_np(rng.standard_normal((m, n)).astype(np.float32) * 0.02)
    x = bits_np(rng.standard_normal((tokens, n)).astype(np.float32))
    data, offsets, minima = p12.pack(w)
    table = p12.tag(offsets, minima)
    outs = []
    for packed in (False, True):
        wd = dev(data) if packed else dev(w.view(np.int16))
        td = dev(table.view(np.int32)) if packed else None
        xd = dev(x.view(np.int16))
        y = torch.empty(tokens * m, dtype=torch.float32, device="cuda")
        assert lib.plamo_kernel_gemm(ptr(wd), ptr(td) if td is not None else 0, ptr(xd), ptr(y), n, m, tokens, 0,
                                     0) == 0
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy().reshape(tokens, m))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    ref = (torch.from_numpy(bf_np(x)).double() @ torch.from_numpy(bf_np(w)).double().T).numpy()
    tol = np.abs(ref) * 2 ** -7 + 1e-5
    assert np.all(np.abs(outs[0] - ref) <= tol)


def test_gemm_swiglu_matches_fp32_and_packed(lib):
    """out_mode 3: the gate_up GEMM with the `swiglu` epilogue (Kernels.metal:202-210):
    y = roundbf(roundbf(g / (1 + exp(-g))) * u) with g, u the BF16-rounded projections."""
    m, n, tokens = 12288, 1536, 70
    rng = np.random.default_rng(7)
    w = bits_np(rng.standard_normal((m, n)).astype(np.float32) * 0.02)
    x = bits_np(rng.standard_normal((tokens, n)).astype(np.float32))
    data, offsets, minima = p12.pack(w)
    table = p12.tag(offsets, minima)
    outs = []
    for packed in (False, True):
        wd = dev(data) if packed else dev(w.view(np.int16))
        td = dev(table.view(np.int32)) if packed else None
        xd = dev(x.view(np.int16))
        y = torch.empty(tokens * 6144, dtype=torch.int16, device="cuda")
        assert lib.plamo_kernel_gemm(ptr(wd), ptr(td) if td is not None else 0, ptr(xd), ptr(y), n, m, tokens, 3,
                                     0) == 0
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy().view(np.uint16).reshape(tokens, 6144))
    assert np.array_equal(outs[0], outs[1])
    ref = (torch.from_numpy(bf_np(x)).double() @ torch.from_numpy(bf_np(w)).double().T).numpy()
    g = roundbf_np(ref[:, :6144].astype(np.float32))
    u = roundbf_np(ref[:, 6144:].astype(np.float32))
    want = roundbf_np(roundbf_np(g / (np.float32(1) + np.exp(-g))) * u)
    got = bf_np(outs[0])
    assert np.all(np.abs(got - want) <= np.abs(want) * 2 ** -6 + 1e-6)
    assert np.mean(got != want) < 0.02
