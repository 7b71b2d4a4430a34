"""Order-exact restatement of the decode step (test infrastructure only).

The semantic oracle (oracle/model.py) sums in torch's order.  On this random-init model the
network amplifies BF16 rounding-path differences: two CPU oracles that differ only in
dot-product summation order disagree by RMSE ~0.013 on the logits, above the 5e-3 the task
sets.  Bitwise comparison is therefore the meaningful check, and it needs the exact
reduction trees of the GPU kernels, restated here in numpy FP32 (every operation is a
correctly rounded IEEE FP32 operation, exactly as on the device, except the GEMV steps):

* GEMV (decode `linear`, Kernels.metal:92-114): lane l of a 64-wide wave owns columns
  it*512 + l*8 .. +8; it accumulates them as v_dot2_f32_bf16 steps over the column pairs in
  order (each step folds two exact BF16 x BF16 products into the FP32 accumulator by the
  MFMA accumulation rule with a group of two: csrc/mfma_model.h, pinned by device vectors in
  tests/golden/dot2_accumulate.npz); the 64 lane sums are combined by an XOR butterfly
  (offsets 32,16,8,4,2,1).  Restated in C (csrc/exact_gemv.c); the library must be built.
* RMSNorm (`norm`, Kernels.metal:46-90): thread t of 256 sums squares of elements 6t..6t+5
  in order; wave butterfly; then (w0+w1)+(w2+w3).  r = 1/sqrt(sum/n + 1e-6).
* q/k norm (`qkv`, Kernels.metal:236-246): 16 lanes x 8 elements (the RoPE pairs d, d+64
  of 4 consecutive d), 16-lane butterfly.
* decode attention (Kernels.metal:440-562 split form): 64-key partitions; score = four
  32-dim chains of q*k (v_dot2_f32_bf16 steps over the dim pairs in order) summed as
  (c0 + c1) + (c2 + c3); softmax statistics per partition with `exp_det`; P.V as two
  chains of fused multiply-adds over keys 0..31 and 32..63 per dim, added at the end;
  merge over partitions in order, in blocks of 128 partitions past 128 (each block summed in
  partition order, the block sums added in block order).
* `exp_det`: Cody-Waite reduction with a 16-bit ln2 head, degree-7 Taylor polynomial, exact
  2^k scale -- the same operation sequence as the device helper.

Pinned by: bit equality with the GPU on the kernel-level entry points, and agreement with the
semantic oracle within the measured noise floor (tests/test_oracle_exact.py).
"""
import numpy as np

from .bf16 import bf_np, bits_np, roundbf_np
from . import rope

F = np.float32
SCALE = F(0.08838834764831845)
EPS = F(1e-6)
WINDOW = 2048
KP = 64
MERGE_BLOCK = 128  # partitions per block of the partition merge (attn_merge_kernel)


def exp_det(x):
    """Device exp_det on an FP32 array (same operation sequence, no contraction)."""
    x = np.asarray(x, dtype=F)
    out = np.zeros_like(x)
    with np.errstate(over="ignore", invalid="ignore"):
        ok = x > F(-80.0)
        big = x > F(88.72283935546875)
        xs = np.where(ok & ~big, x, F(0))
        k = np.rint(xs * F(1.44269502162933349609375)).astype(F)
        r = ((xs - k * F(0.693145751953125)) - k * F(1.428606765330187e-06)).astype(F)
        p = F(1.98412698e-04)
        for c in (F(1.38888889e-03), F(8.33333377e-03), F(4.16666679e-02), F(1.66666672e-01), F(0.5), F(1.0),
                  F(1.0)):
            p = (p * r + c).astype(F)
        v = np.ldexp(p, k.astype(np.int32)).astype(F)
    out = np.where(ok, v, F(0))
    out = np.where(big, F(np.inf), out)
    return out.astype(F)


def butterfly(a):
    """XOR butterfly over the last axis (64 or 16 lanes); returns lane 0."""
    n = a.shape[-1]
    idx = np.arange(n)
    o = n // 2
    while o:
        a = (a + a[..., idx ^ o]).astype(F)
        o //= 2
    return a[..., 0]


_C = None


def _c_lib():
    """oracle/_lib/libexact.so (built by `make -C oracle`), or None."""
    global _C
    if _C is None:
        import ctypes
        import os
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libexact.so")
        _C = False
        if os.path.exists(path):
            lib = ctypes.CDLL(path)
            lib.plamo_oracle_gemv.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 2
            lib.plamo_oracle_dot2_chain.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 2 + [ctypes.c_int32]
            lib.plamo_oracle_attn_scores.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_int64, ctypes.c_void_p]
            lib.plamo_oracle_attn_pv.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_int64, ctypes.c_void_p]
            _C = lib
    return _C or None


def _lib():
    lib = _c_lib()
    if lib is None:
        raise RuntimeError("oracle C restatement not built (make -C oracle)")
    return lib


def gemv(w, x):
    """W [m, n] FP32 (BF16 values), x [n] -> FP32 [m] in the kernel's order
    (csrc/exact_gemv.c)."""
    m, n = w.shape
    assert n % 512 == 0
    w = np.ascontiguousarray(w, dtype=F)
    x = np.ascontiguousarray(x, dtype=F)
    y = np.empty(m, F)
    _lib().plamo_oracle_gemv(w.ctypes.data, x.ctypes.data, y.ctypes.data, m, n)
    return y


def attn_scores(q, keys):
    """q [16][128], keys [n][128] (BF16-valued FP32) -> raw scores [16][n] in the decode
    attention kernel's order (csrc/exact_gemv.c)."""
    qb = bits_np(np.ascontiguousarray(q, dtype=F))
    kb = bits_np(np.ascontiguousarray(keys, dtype=F))
    assert np.array_equal(bf_np(qb), q) and np.array_equal(bf_np(kb), keys), "BF16 values expected"
    n = kb.shape[0]
    out = np.empty((16, n), F)
    _lib().plamo_oracle_attn_scores(qb.ctypes.data, kb.ctypes.data, n, out.ctypes.data)
    return out


def attn_pv(e, v_bits):
    """One partition's P.V: e [16][64] FP32, v_bits [nk][128] BF16 bits -> [16][128] in the
    decode attention kernel's order (two 32-key chains of fused multiply-adds per head and
    dim, then their sum; csrc/exact_gemv.c)."""
    e = np.ascontiguousarray(e, dtype=F)
    assert e.shape == (16, 64)
    vb = np.ascontiguousarray(v_bits, dtype=np.uint16)
    out = np.empty((16, 128), F)
    _lib().plamo_oracle_attn_pv(e.ctypes.data, vb.ctypes.data, vb.shape[0], out.ctypes.data)
    return out


def dot2_chain(a_pairs, b_pairs, acc, fast=True):
    """v_dot2_f32_bf16 chains: a, b uint32 BF16 pairs (low half first) [steps][n], acc [n]
    -> every intermediate accumulator [steps][n].  fast=False uses the general fold."""
    a = np.ascontiguousarray(a_pairs, dtype=np.uint32)
    b = np.ascontiguousarray(b_pairs, dtype=np.uint32)
    c = np.ascontiguousarray(acc, dtype=F)
    steps, n = a.shape
    out = np.empty((steps, n), F)
    _lib().plamo_oracle_dot2_chain(a.ctypes.data, b.ctypes.data, c.ctypes.data, out.ctypes.data, n, steps,
                                   1 if fast else 0)
    return out


def block_sumsq(v):
    """256-thread sum of squares of a 1536 vector: thread t sums the squares of elements
    6t .. 6t+5 in order, then the wave butterfly, then (w0 + w1) + (w2 + w3)."""
    t = v.astype(F).reshape(256, 6)
    ss = np.zeros(256, F)
    for k in range(6):
        ss += t[:, k] * t[:, k]
    w = butterfly(ss.reshape(4, 64))
    return F(F(w[0] + w[1]) + F(w[2] + w[3]))


def gain(w_bits, offset):
    return roundbf_np((bf_np(w_bits) + F(offset)).astype(F))


def norm_rows(x, w_bits, offset):
    r = F(1) / np.sqrt(F(block_sumsq(x) / F(1536)) + EPS)
    return roundbf_np(roundbf_np(x * r) * gain(w_bits, offset))


def head_norm(v, w_bits):
    """q/k RMSNorm over 128, +1 offset: lane `sub` of 16 sums the squares of dims
    sub*4+j then 64+sub*4+j (j = 0..3) in that order; 16-lane XOR butterfly."""
    v = v.astype(F)
    lanes = np.concatenate([v[:64].reshape(16, 4), v[64:].reshape(16, 4)], axis=1)
    ss = np.zeros(16, F)
    for j in range(8):
        ss += lanes[:, j] * lanes[:, j]
    tot = butterfly(ss[None, :])[0]
    r = F(1) / np.sqrt(F(tot / F(128)) + EPS)
    return roundbf_np(roundbf_np(v * r) * gain(w_bits, 1.0))


def rope_pair(z, c, s):
    """z [..., 128]; c, s [..., 64] -> rotated (Kernels.metal:261-274)."""
    a, b = z[..., :64], z[..., 64:]
    ra = roundbf_np(roundbf_np(a * c) + roundbf_np(-b * s))
    rb = roundbf_np(roundbf_np(b * c) + roundbf_np(a * s))
    return np.concatenate([ra, rb], -1)


class ExactDecoder:
    """Bit-exact CPU twin of the decode step (one sequence)."""

    def __init__(self, weights, context, local_capacity, qsa=None):
        # qsa: the QSA indexers of the global layers (oracle.adapters.QsaTwin), None: dense
        self.qsa = qsa
        self.w = weights
        self.context = context
        self.cap = [context if i % 8 == 7 else local_capacity for i in range(16)]
        self.layers = []
        for L in weights.layers:
            self.layers.append({k: (v.numpy() if hasattr(v, "numpy") else v) for k, v in L.items()})
        self.head = weights.head.numpy()
        self.final = weights.final.numpy()
        lc, ls = rope.local_table(weights.f_local, 2064)
        gc, gs = rope.global_table(weights.f_full, context)
        self.lc, self.ls, self.gc, self.gs = lc, ls, gc, gs
        self.keys = [np.zeros((c, 128), np.uint16) for c in self.cap]
        self.values = [np.zeros((c, 128), np.uint16) for c in self.cap]

    def _bits(self, t):
        return np.asarray(t, dtype=np.int64).astype(np.uint16)

    def attention(self, layer, qkv, pos, mask=None):
        """mask (global layers with QSA): bool per complete block of four keys, the selected
        ones; keys of the unfinished block are always seen."""
        full = layer % 8 == 7
        cap = self.cap[layer]
        L = self.layers[layer]
        first = 0 if full else max(0, pos - (WINDOW - 1))
        count = pos + 1 - first
        z = np.stack([head_norm(qkv[h * 128:(h + 1) * 128], self._bits(L["q_norm"])) for h in range(16)])
        zk = head_norm(qkv[2048:2176], self._bits(L["k_norm"]))
        qc = pos if full else pos - first
        c, s = (self.gc[qc], self.gs[qc]) if full else (self.lc[qc], self.ls[qc])
        q = rope_pair(z, c[None], s[None])
        knew = rope_pair(zk, self.gc[pos], self.gs[pos]) if full else zk
        slot = pos % cap
        self.keys[layer][slot] = bits_np(knew)
        self.values[layer][slot] = bits_np(qkv[2176:2304])
        start = first % cap
        r = np.arange(count)
        phys = (start + r) % cap
        keys = bf_np(self.keys[layer][phys])
        if not full:
            keys = rope_pair(keys, self.lc[r], self.ls[r])
        vbits = self.values[layer][phys]
        scores = attn_scores(q, keys)
        parts = (count + KP - 1) // KP
        pm = np.zeros((parts, 16), F)
        pl = np.zeros((parts, 16), F)
        po = np.zeros((parts, 16, 128), F)
        if mask is not None and len(mask) > 0:
            seen = (r // 4 >= len(mask)) | np.asarray(mask, bool)[np.minimum(r // 4, len(mask) - 1)]
        else:
            mask = None
        for p in range(parts):
            k0 = p * KP
            kk = keys[k0:k0 + KP]
            nk = kk.shape[0]
            sc = (scores[:, k0:k0 + nk] * SCALE).astype(F)
            full_sc = np.full((16, 64), -np.inf, F)
            full_sc[:, :nk] = sc
            if mask is not None:
                full_sc[:, :nk][:, ~seen[k0:k0 + nk]] = -np.inf
            m = full_sc.max(1)
            e = np.zeros((16, 64), F)
            with np.errstate(invalid="ignore"):
                e[:, :nk] = np.where(np.isfinite(full_sc[:, :nk]), exp_det(full_sc[:, :nk] - m[:, None]), F(0))
            pm[p], pl[p] = m, butterfly(e)
            po[p] = attn_pv(e, vbits[k0:k0 + KP])
        # merge: M = max m_p; w_p = exp(m_p - M); num = sum o_p w_p, den = sum l_p w_p as
        # sums of blocks of MERGE_BLOCK partitions (each in partition order, from 0), added in
        # block order (one block: the plain partition-order sum)
        M = pm.max(0)
        num = np.zeros((16, 128), F)
        den = np.zeros(16, F)
        for b0 in range(0, parts, MERGE_BLOCK):
            bnum = np.zeros((16, 128), F)
            bden = np.zeros(16, F)
            for p in range(b0, min(b0 + MERGE_BLOCK, parts)):
                wgt = exp_det(pm[p] - M)
                bden = (bden + pl[p] * wgt).astype(F)
                bnum = (bnum + po[p] * wgt[:, None]).astype(F)
            den = (den + bden).astype(F)
            num = (num + bnum).astype(F)
        return roundbf_np((num / den[:, None]).astype(F)).reshape(2048)

    def step(self, token, pos, x_prev=None, d_prev=None):
        """One decode step; returns (logit_bits, hidden, next)."""
        Ls = self.layers
        emb = bf_np(self.w.embed_bits[token])
        x = emb.astype(F)
        xn = norm_rows(x, self._bits(Ls[0]["pre"]), 1.0)
        d = None
        post_mlp = F(1 / 5.0 ** 1.5)
        for i, L in enumerate(Ls):
            if i > 0:
                z = norm_rows(d, self._bits(Ls[i - 1]["post_mlp"]), post_mlp)
                x = roundbf_np(x + z)
                xn = norm_rows(x, self._bits(L["pre"]), 1.0)
            qkv = roundbf_np(gemv(L["qkv"], xn))
            mask = self.qsa.decode_mask(self, i, xn, pos) if (self.qsa is not None and i % 8 == 7) else None
            att = self.attention(i, qkv, pos, mask)
            o = roundbf_np(gemv(L["o"], att))
            z = norm_rows(o, self._bits(L["post"]), 0.2)
            x = roundbf_np(x + z)
            xn = norm_rows(x, self._bits(L["pre_mlp"]), 1.0)
            gu = gemv(L["up"], xn)
            g, u = roundbf_np(gu[:6144]), roundbf_np(gu[6144:])
            act = roundbf_np(roundbf_np(g / (F(1) + exp_det(-g))) * u)
            d = roundbf_np(gemv(L["down"], act))
        return self.head_step(d, x)

    def head_step(self, d, x):
        """The head of a step: last layer's post-norm and residual, final norm, LM head GEMV
        -> (logit_bits, hidden, next)."""
        z = norm_rows(d, self._bits(self.layers[15]["post_mlp"]), F(1 / 5.0 ** 1.5))
        x = roundbf_np(x + z)
        h = norm_rows(x, self._bits(self.final), 1.0)
        logits = gemv(self.head, h)
        lb = bits_np(logits)
        from .sampler import argmax_gpu
        return lb, h, argmax_gpu(bf_np(lb))
