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
