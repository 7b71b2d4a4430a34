"""Order-exact restatement of the trained adapters (test infrastructure only): the MTP
draft (Runtime.draft, Runtime.swift:485-520) in the arithmetic of the gfx950 kernels, and a
textbook FP64 version of the same formula that pins it.

MTP draft after token `first`, from the first output row's normalised hidden state h:
  x = [h | embedding(first)]                                  (3072, Runtime.swift:493-494)
  u = roundbf(W_up x)            the decode GEMV's order (exact.gemv: lanes own 8 columns of
                                 each 512-column step, v_dot2 steps, XOR butterfly)
  a = roundbf(u / (1 + exp(-u)))                               (mtp_activate, Kernels.metal:347-350)
  y = roundbf(W_down a)          mtp_down_kernel's order: lane l of a 64-lane wave owns columns
                                 4l .. 4l+3, two v_dot2 steps over the pairs, XOR butterfly
  z = roundbf(x[:1536] + y)                                    (mtp_add, Kernels.metal:352-356)
  draft = first maximum of the BF16 logits of the LM head on z (Runtime.swift:502-503)

Pinned by: bit equality with the GPU draft (tests/test_gpu_adapters.py), and agreement with
`textbook_draft` (FP64 sums, exact exp) within the rounding of its BF16 steps
(tests/test_oracle_adapters.py).

QSA indexers (Runtime.swift:378-418, Kernels.metal:564-702), QsaTwin, on each global layer:
  p    = roundbf(P xn)           the indexer projection [640] of the pre-attention normed row
                                 (decode: the GEMV order; prefill: the MFMA GEMM order)
  q_h  = rope(norm(p[128h:128h+128], q_norm), pos)   h = 0..3, global RoPE
  raw[pos] = p[512:640]
  block b (complete once 4b + 3 is written): mean_d = roundbf((((k0 + k1) + k2) + k3) / 4)
         over raw[4b..4b+3], pooled[b] = rope(norm(mean, k_norm), 4b)
  norm(v, w): lane l of a wave holds (v_l, v_l+64), ss = butterfly(v_l^2 + v_l+64^2),
         r = 1 / sqrt(ss / 128 + 1e-6), z = roundbf(roundbf(v r) roundbf(w + 1))
  score(b) = (sum over h in order of max(0, q_h . pooled[b])) / sqrt(128), each dot product
         one v_dot2 chain over the 64 dimension pairs in order
  selection: with C = (pos + 1) / 4 complete blocks and k = min(C, budget / 4), every block
         if k == C, else the k largest max(score, 0), ties to the lower index (a sort here;
         a radix search on the device)
  attention then sees the selected blocks and the keys of the unfinished block.

Pinned by: the reference's selection known-answer test (QSATests.swift:6-46) restated over
`select`, a textbook FP64 indexer (`textbook_scores`) within BF16 rounding, and bit equality of
decode and prefill with the GPU (tests/test_gpu_qsa.py).
"""
import os

import numpy as np

from . import exact
from .bf16 import bf_np, bits_np, roundbf_np
from .model import read_safetensors

F = np.float32
MTP_RANK = 256


class Adapters:
    """BF16 bits of auxiliary.safetensors (Auxiliary.swift:72-111)."""

    def __init__(self, directory):
        raw = read_safetensors(os.path.join(directory, "auxiliary.safetensors"))
        self.mtp_up = raw["mtp.heads.0.up.weight"]        # [256][3072]
        self.mtp_down = raw["mtp.heads.0.down.weight"]    # [1536][256]
        self.qsa = {l: {"proj": raw[f"qsa.{l}.proj.weight"], "q_norm": raw[f"qsa.{l}.q_norm.weight"],
                        "k_norm": raw[f"qsa.{l}.k_norm.weight"]} for l in (7, 15)}


def _pairs(v_bits):
    """[..., 2k] BF16 bits -> [..., k] uint32 pairs (element 2k in the low half)."""
    v = np.asarray(v_bits, dtype=np.uint32)
    return v[..., 0::2] | (v[..., 1::2] << 16)


def mtp_down(w_bits, a):
    """W [1536][256] BF16 bits, a [256] BF16-valued -> raw FP32 sums [1536] in the kernel's
    order: lane l accumulates pairs (4l, 4l+1) then (4l+2, 4l+3) from 0, then the butterfly."""
    rows = w_bits.shape[0]
    wp = _pairs(w_bits).reshape(rows, 64, 2)                  # [row][lane][step]
    ap = _pairs(bits_np(np.asarray(a, F))).reshape(64, 2)     # [lane][step]
    wa = np.ascontiguousarray(wp.transpose(2, 0, 1).reshape(2, rows * 64))
    aa = np.ascontiguousarray(np.broadcast_to(ap.T[:, None, :], (2, rows, 64)).reshape(2, rows * 64))
    acc = exact.dot2_chain(wa, aa, np.zeros(rows * 64, F))[-1]
    return exact.butterfly(acc.reshape(rows, 64))


def mtp_draft(ex, adapters, hidden, first):
    """-> (draft logits BF16 bits, draft token) on the decode twin `ex` (its head and
    embedding)."""
    x = np.concatenate([np.asarray(hidden, F), bf_np(ex.w.embed_bits[first]).astype(F)])
    u = roundbf_np(exact.gemv(bf_np(adapters.mtp_up).astype(F), x))
    a = roundbf_np((u / (F(1) + exact.exp_det(-u))).astype(F))
    y = roundbf_np(mtp_down(adapters.mtp_down, a))
    z = roundbf_np((x[:1536] + y).astype(F))
    logits = exact.gemv(ex.head, z)
    lb = bits_np(logits)
    from .sampler import argmax_gpu
    return lb, argmax_gpu(bf_np(lb))


def textbook_draft(embed_bits, head, adapters, hidden, first):
    """The same formula with FP64 sums and exp, rounding to BF16 only where the reference
    stores BF16 (-> FP64 logits of the head)."""
    x = np.concatenate([np.asarray(hidden, np.float64), bf_np(embed_bits[first]).astype(np.float64)])
    u = bf_np(bits_np((bf_np(adapters.mtp_up).astype(np.float64) @ x).astype(F))).astype(np.float64)
    a = bf_np(bits_np((u / (1 + np.exp(-u))).astype(F))).astype(np.float64)
    y = bf_np(bits_np((bf_np(adapters.mtp_down).astype(np.float64) @ a).astype(F))).astype(np.float64)
    z = bf_np(bits_np((x[:1536] + y).astype(F))).astype(np.float64)
    return np.asarray(head, np.float64) @ z


QSA_SCALE = F(0.08838834764831845)


def qsa_norm_rope(v, w_bits, c, s):
    """The indexer's head RMSNorm (gain w + 1) and global RoPE with table rows c, s."""
    v = np.asarray(v, F)
    a, b = v[:64], v[64:]
    ss = exact.butterfly(((a * a) + (b * b)).astype(F)[None])[0]
    r = F(1) / np.sqrt(F(ss / F(128)) + exact.EPS)
    z = roundbf_np(roundbf_np(v * r) * exact.gain(w_bits, 1.0))
    return exact.rope_pair(z, c, s)


def select(scores, complete, budget):
    """Blocks chosen among `complete` (bool [complete]): the budget/4 largest max(score, 0),
    ties to the lower index; all of them when the budget covers them."""
    k = min(complete, budget // 4)
    chosen = np.zeros(complete, bool)
    if k == complete:
        chosen[:] = True
        return chosen
    s = np.asarray(scores[:complete], F)
    val = np.where(s > 0, s, F(0)).astype(F).view(np.uint32).astype(np.int64)
    order = np.lexsort((np.arange(complete), -val))
    chosen[order[:k]] = True
    return chosen


class QsaTwin:
    """Indexer state of the global layers (raw and pooled keys) and the order-exact selection.
    Attach to exact.ExactDecoder(qsa=...); the prefill twin uses the decoder's."""

    def __init__(self, adapters, context, budget):
        self.budget = budget
        self.blocks = context // 4
        self.words = (self.blocks + 31) // 32
        self.a = adapters
        self.proj = {l: bf_np(adapters.qsa[l]["proj"]).astype(F) for l in adapters.qsa}
        self.raw = {l: np.zeros((context, 128), np.uint16) for l in adapters.qsa}
        self.pooled = {l: np.zeros((max(self.blocks, 1), 128), np.uint16) for l in adapters.qsa}
        self.last_scores = {}

    def _rows(self, ex, layer, proj, p0):
        """proj [T][640] BF16-valued rows of positions p0 .. p0+T-1 -> uint32 masks [T][words]
        (bit b of word b / 32: block b selected)."""
        A = self.a.qsa[layer]
        qn, kn = np.asarray(A["q_norm"], np.uint16), np.asarray(A["k_norm"], np.uint16)
        T = proj.shape[0]
        raw, pooled = self.raw[layer], self.pooled[layer]
        queries = np.empty((T, 4, 128), np.uint16)
        for t in range(T):
            pos = p0 + t
            for h in range(4):
                queries[t, h] = bits_np(qsa_norm_rope(proj[t, 128 * h:128 * h + 128], qn, ex.gc[pos], ex.gs[pos]))
            raw[pos] = bits_np(proj[t, 512:640])
        for b in range(p0 // 4, (p0 + T) // 4):
            k = bf_np(raw[4 * b:4 * b + 4]).astype(F)
            mean = roundbf_np(((((k[0] + k[1]) + k[2]) + k[3]) / F(4)).astype(F))
            pooled[b] = bits_np(qsa_norm_rope(mean, kn, ex.gc[4 * b], ex.gs[4 * b]))
        masks = np.zeros((T, max(self.words, 1)), np.uint32)
        self.last_scores[layer] = []
        for t in range(T):
            complete = (p0 + t + 1) // 4
            if complete == 0:
                self.last_scores[layer].append(np.zeros(0, F))
                continue
            kp = _pairs(pooled[:complete])                                   # [C][64]
            score = np.zeros(complete, F)
            for h in range(4):
                qp = _pairs(queries[t, h])                                   # [64]
                a = np.ascontiguousarray(np.broadcast_to(qp[:, None], (64, complete)))
                acc = exact.dot2_chain(a, np.ascontiguousarray(kp.T), np.zeros(complete, F))[-1]
                score = (score + np.maximum(acc, F(0))).astype(F)
            score = (score * QSA_SCALE).astype(F)
            self.last_scores[layer].append(score)
            chosen = np.flatnonzero(select(score, complete, self.budget))
            np.bitwise_or.at(masks[t], chosen >> 5, (np.uint32(1) << (chosen & 31).astype(np.uint32)))
        return masks

    def decode_mask(self, ex, layer, xn, pos):
        """One decode step: bool [complete blocks] for exact.ExactDecoder.attention."""
        p = roundbf_np(exact.gemv(self.proj[layer], xn))
        m = self._rows(ex, layer, p[None], pos)[0]
        complete = (pos + 1) // 4
        return ((m[np.arange(complete) >> 5] >> (np.arange(complete) & 31).astype(np.uint32)) & 1).astype(bool)

    def prefill_masks(self, ex, layer, xn, p0):
        """A prefill chunk's rows xn [T][1536] -> masks [T][words] for exact_prefill.flash."""
        from .exact_prefill import mfma_gemm
        p = roundbf_np(mfma_gemm(bits_np(self.proj[layer]), bits_np(xn)))
        return self._rows(ex, layer, p, p0)


def textbook_scores(adapters, layer, gcos, gsin, rows, relu=True, gain_offset=1.0, k_rope_shift=0):
    """FP64 indexer scores of every query row against the blocks complete at its position,
    from the projected rows of positions 0 .. T-1 (BF16-valued [T][640]): the same formula with
    exact sums and square roots.  relu, gain_offset and k_rope_shift (block keys rotated at
    4b + shift) exist to plant mistakes that a check against this function must catch."""
    A = adapters.qsa[layer]
    gq = bf_np(np.asarray(A["q_norm"], np.uint16)).astype(np.float64) + gain_offset
    gk = bf_np(np.asarray(A["k_norm"], np.uint16)).astype(np.float64) + gain_offset

    def nr(v, g, c, s):
        v = np.asarray(v, np.float64)
        z = v / np.sqrt(np.mean(v * v) + 1e-6) * g
        c, s = np.asarray(c, np.float64), np.asarray(s, np.float64)
        return np.concatenate([z[:64] * c - z[64:] * s, z[64:] * c + z[:64] * s])

    rows = np.asarray(rows, np.float64)
    blocks = len(rows) // 4
    pk = [nr(rows[4 * b:4 * b + 4, 512:].mean(0), gk, gcos[4 * b + k_rope_shift], gsin[4 * b + k_rope_shift])
          for b in range(blocks)]
    out = []
    for pos in range(len(rows)):
        qs = [nr(rows[pos, 128 * h:128 * h + 128], gq, gcos[pos], gsin[pos]) for h in range(4)]
        act = (lambda v: max(0.0, v)) if relu else (lambda v: v)
        out.append(np.array([sum(act(float(q @ k)) for q in qs) / np.sqrt(128) for k in pk[:(pos + 1) // 4]]))
    return out
