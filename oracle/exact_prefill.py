"""Order-exact restatement of the MFMA prefill (test infrastructure only).

The prefill of Runtime.prefill (Runtime.swift:469-483: chunks of the prompt through every
layer, K/V written for each chunk, attention over the visible keys, logits of the last token)
in the exact arithmetic of the gfx950 prefill kernels, so that the GPU prefill can be held to
it bit for bit:

* projections (`matrix`, Kernels.metal:149-200): the MFMA accumulation model of
  oracle/csrc/mfma_model.h, K ascending (csrc/exact_gemm.c); outputs rounded to BF16;
* the gate_up epilogue (`swiglu`, Kernels.metal:202-210): bf16(bf16(g / (1 + exp_det(-g))) * u)
  of the BF16-rounded gate and up accumulators;
* row norms (`norm`, Kernels.metal:46-90) of the prefill kernel: lane l of a 64-wide wave
  sums the squares of elements 512c + 8l + j (c = 0..2, j = 0..7) in that order, then the
  wave's XOR butterfly; post-norm, residual add and the next layer's pre-norm as in decode;
* q/k norm and RoPE (`qkv`, Kernels.metal:223-259) as in decode (oracle/exact.py), queries
  of local layers rotated at pos - base of their 16-token chunk (Runtime.swift:389);
* attention (Runtime.swift:389-444): the flash kernel's tiles, parts, softmax with
  `exp2_det` and MFMA chains (csrc/exact_flash.c);
* the last token's head: the decode head (post-norm, residual, final norm, LM head GEMV),
  shared with oracle/exact.py.

Pinned by: device-measured accumulator vectors (tests/golden/mfma_accumulate.npz, written
by tests/golden/make_mfma_fixture.py on the GPU), closed forms and error bounds of the model
(tests/test_oracle_prefill.py), the flash twin against an FP32 softmax within 1 BF16 ulp,
and bit equality with the GPU kernels and the whole GPU prefill (tests/test_gpu_prefill_exact.py).
"""
import ctypes

import numpy as np

from . import exact
from .bf16 import bf_np, bits_np, roundbf_np

F = np.float32
WINDOW = 2048
CHUNK = 16
POST_MIXER = F(0.2)
POST_MLP = F(1 / 5.0 ** 1.5)

_SIGS = {
    "plamo_oracle_mfma_gemm": (None, [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3),
    "plamo_oracle_mfma_chain": (ctypes.c_float, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_float]),
    "plamo_oracle_flash": (None, [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 3 + [ctypes.c_int32, ctypes.c_void_p,
                                                                                  ctypes.c_void_p, ctypes.c_int64]),
    "plamo_oracle_exp2_det": (ctypes.c_float, [ctypes.c_float]),
}


def lib():
    """oracle/_lib/libexact.so with the prefill entry points; raises if it is not built."""
    c = exact._c_lib()
    if c is None:
        raise RuntimeError("oracle C restatement not built (make -C oracle)")
    for name, (res, args) in _SIGS.items():
        fn = getattr(c, name)
        fn.restype, fn.argtypes = res, args
    return c


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


def mfma_gemm(w_bits, x_bits):
    """W [m][k], X [tokens][k] BF16 bits -> raw FP32 accumulators [tokens][m]."""
    w, x = _u16(w_bits), _u16(x_bits)
    m, k = w.shape
    t = x.shape[0]
    assert x.shape[1] == k and k % 8 == 0
    y = np.empty((t, m), F)
    lib().plamo_oracle_mfma_gemm(w.ctypes.data, x.ctypes.data, y.ctypes.data, m, k, t)
    return y


def mfma_chain(a_bits, b_bits, acc=0.0):
    """One accumulator chain over the products a[i] * b[i] (groups of 8 in order)."""
    a, b = _u16(a_bits), _u16(b_bits)
    return F(lib().plamo_oracle_mfma_chain(a.ctypes.data, b.ctypes.data, a.size, float(acc)))


def exp2_det(x):
    c = lib()
    return np.array([c.plamo_oracle_exp2_det(float(v)) for v in np.ravel(x)], F).reshape(np.shape(x))


def flash(q_bits, keys, values, lcos_bits, lsin_bits, capacity, p0, full, qsa_mask=None):
    """q [tokens][16][128], keys/values [capacity][128], local table [rows][64] (BF16 bits)
    -> attention output BF16 bits [tokens][2048].  qsa_mask: uint32 [tokens][words] selected
    blocks of four keys per query (global layers), None: every key."""
    q = _u16(q_bits)
    tokens = q.shape[0]
    k, v = _u16(keys), _u16(values)
    lc, ls = _u16(lcos_bits), _u16(lsin_bits)
    out = np.empty((tokens, 2048), np.uint16)
    m = None if qsa_mask is None else np.ascontiguousarray(qsa_mask, dtype=np.uint32)
    lib().plamo_oracle_flash(q.ctypes.data, k.ctypes.data, v.ctypes.data, lc.ctypes.data, ls.ctypes.data, capacity,
                             p0, tokens, 1 if full else 0, out.ctypes.data, None if m is None else m.ctypes.data,
                             0 if m is None else m.shape[1])
    return out


def _bf16_bits(a):
    """BF16 bits of an FP32 array holding BF16 values (the high halves, no rounding)."""
    u = np.ascontiguousarray(a, dtype=F).view(np.uint32)
    assert not np.any(u & 0xFFFF), "weights must be BF16 values"
    return (u >> 16).astype(np.uint16)


def rows_sumsq(v):
    """Prefill row sums of squares, [n][1536] -> [n]: lane l of 64 sums elements 512c + 8l + j
    (c-major, then j) in order, then the XOR butterfly."""
    n = v.shape[0]
    lanes = v.astype(F).reshape(n, 3, 64, 8).transpose(0, 2, 1, 3).reshape(n, 64, 24)
    ss = np.zeros((n, 64), F)
    for j in range(24):
        ss = (ss + lanes[:, :, j] * lanes[:, :, j]).astype(F)
    return exact.butterfly(ss)


def rows_norm(x, g_bits, offset):
    r = (F(1) / np.sqrt((rows_sumsq(x) / F(1536)).astype(F) + exact.EPS)).astype(F)
    return roundbf_np(roundbf_np(x * r[:, None]) * exact.gain(g_bits, offset)[None, :])


class ExactPrefill:
    """Prefill twin sharing the KV cache (and the weights and RoPE tables) of an
    exact.ExactDecoder, so decode steps can follow a prefill on the same state."""

    def __init__(self, decoder, chunk=2048):
        self.ex = decoder
        self.chunk = min(chunk, (decoder.context + CHUNK - 1) // CHUNK * CHUNK)
        self.wb = [{k: _bf16_bits(L[k]) for k in ("qkv", "o", "up", "down")} for L in decoder.layers]
        self.lcb, self.lsb = bits_np(decoder.lc), bits_np(decoder.ls)

    def _bits(self, t):
        return self.ex._bits(t)

    def prefill(self, tokens, p0=0, kv_layers=None):
        """Runtime.prefill from position p0 -> (logit_bits, hidden, next) of the last token.
        kv_layers = L < 16: every chunk stops once layer L - 1 has written its keys and
        values (layers 0 .. L - 2 in full), and the call returns None.  Layer i's keys and
        values depend only on layers 0 .. i of this and earlier chunks, so the cached rows of
        layers 0 .. L - 1 are those of the full prefill."""
        out = None
        for c0 in range(0, len(tokens), self.chunk):
            part = tokens[c0:c0 + self.chunk]
            out = self._chunk(part, p0 + c0, c0 + len(part) == len(tokens), kv_layers)
        return out

    def _qk_prep(self, layer, qkv, p0):
        ex = self.ex
        L = ex.layers[layer]
        full = layer % 8 == 7
        cap = ex.cap[layer]
        n = qkv.shape[0]
        q16 = np.empty((n, 16, 128), np.uint16)
        for t in range(n):
            pos = p0 + t
            chunk = p0 + (t // CHUNK) * CHUNK
            base = max(0, chunk - (WINDOW - 1))
            qc = pos if full else pos - base
            c, s = (ex.gc[qc], ex.gs[qc]) if full else (ex.lc[qc], ex.ls[qc])
            z = np.stack([exact.head_norm(qkv[t, h * 128:(h + 1) * 128], self._bits(L["q_norm"])) for h in range(16)])
            q16[t] = bits_np(exact.rope_pair(z, c[None], s[None]))
            zk = exact.head_norm(qkv[t, 2048:2176], self._bits(L["k_norm"]))
            if full:
                zk = exact.rope_pair(zk, ex.gc[pos], ex.gs[pos])
            ex.keys[layer][pos % cap] = bits_np(zk)
            ex.values[layer][pos % cap] = bits_np(qkv[t, 2176:2304])
        return q16

    def _chunk(self, tokens, p0, last, kv_layers=None):
        ex = self.ex
        Ls = ex.layers
        emb = bf_np(ex.w.embed_bits[np.asarray(tokens, np.int64)]).astype(F)
        x = emb
        xn = rows_norm(x, self._bits(Ls[0]["pre"]), 1.0)
        d = None
        for i, L in enumerate(Ls):
            full = i % 8 == 7
            if i > 0:
                z = rows_norm(d, self._bits(Ls[i - 1]["post_mlp"]), POST_MLP)
                x = roundbf_np(x + z)
                xn = rows_norm(x, self._bits(L["pre"]), 1.0)
            qkv = roundbf_np(mfma_gemm(self.wb[i]["qkv"], bits_np(xn)))
            q16 = self._qk_prep(i, qkv, p0)
            if kv_layers is not None and i + 1 >= kv_layers:
                return None
            mask = ex.qsa.prefill_masks(ex, i, xn, p0) if (ex.qsa is not None and full) else None
            att = flash(q16, ex.keys[i], ex.values[i], self.lcb, self.lsb, ex.cap[i], p0, full, mask)
            o = roundbf_np(mfma_gemm(self.wb[i]["o"], att))
            z = rows_norm(o, self._bits(L["post"]), POST_MIXER)
            x = roundbf_np(x + z)
            xn = rows_norm(x, self._bits(L["pre_mlp"]), 1.0)
            gu = mfma_gemm(self.wb[i]["up"], bits_np(xn))
            g, u = roundbf_np(gu[:, :6144]), roundbf_np(gu[:, 6144:])
            act = roundbf_np(roundbf_np(g / (F(1) + exact.exp_det(-g))) * u)
            d = roundbf_np(mfma_gemm(self.wb[i]["down"], bits_np(act)))
        if not last:
            return None
        return ex.head_step(d[-1], x[-1])
