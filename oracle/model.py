"""PLaMo-3 0.8B forward pass on the CPU (test infrastructure only).

``Oracle`` restates ``Runtime.forward``/``prefill`` (Sources/Plamo/Runtime.swift:327-483) with
the arithmetic of the Metal kernels it dispatches, in PyTorch-CPU FP32 with a BF16
round-to-nearest-even (``roundbf``) at exactly the reference's points:

* ``norm``      Kernels.metal:46-90   ``roundbf(roundbf(x*r) * roundbf(bf(w)+offset))``,
                ``r = 1/sqrt(mean(x^2)+1e-6)``; residual ``roundbf(res+z)``.
* ``linear``/``matrix``  Kernels.metal:92-114,149-200  ``roundbf(W.x)``; the LM head keeps
                BF16 bits (``full == 2``).
* ``qkv``       Kernels.metal:223-259  128-wide q/k norm (+1 offset), rotate-half RoPE; global
                keys rotated at the absolute position, local keys cached normalised but
                unrotated; K/V written to slot ``pos % capacity``.
* attention     Runtime.swift:389-444 with ``rotate`` (277-285), ``matrix`` scores, ``softmax``
                (358-397: scale 1/sqrt(128) before the max, window ``[end-2048, end)``) and
                ``attend`` (400-437: ``roundbf(sum p.v)``).  Local keys take chunk-relative
                coordinates ``r`` from ``base = max(0, chunk_start-2047)``; local queries take
                ``pos-base``.
* ``swiglu``    Kernels.metal:202-210.
* schedule      Runtime.swift:376-458 (offsets 1.0 / 0.2 / 5^-1.5; fused next norm),
                16-token prefill chunks (Runtime.swift:129,476).

Reduction order is torch's, so this is the *semantic* oracle: the GPU is compared to it
with the tolerances of the task (logits max-abs 2e-2, RMSE 5e-3) and exact greedy IDs.

Pinning (tests/test_oracle_model.py): every kernel-level function is pinned by the
reference's kernel tests restated on the CPU (closed-form window mean of
PlamoTests.swift:156-194, fused norm == separate norm of PlamoTests.swift:288-325, brute-force
GEMV of PlamoTests.swift:327-364); the assembled forward is pinned against ``textbook_logits``,
an independent FP32 implementation written from the HF/MLX layer algorithm
(scripts/verify_long.py:24-56, scripts/auxiliary.py:35-47) with no intermediate BF16
rounding, using the reference's own acceptance rule (argmax equal, cosine > 0.999,
RMSE < 0.2; scripts/verify.py:62-63, verify_long.py:116).
"""
import json
import os

import numpy as np
import torch

from .bf16 import bf_t, bits_t, roundbf_t
from . import rope

HIDDEN, HEADS, HEAD_DIM, INTER, VOCAB, LAYERS = 1536, 16, 128, 6144, 107520, 16
WINDOW = 2048
SCALE = np.float32(0.08838834764831845)
POST_MLP_OFFSET = float(np.float32(1 / 5.0 ** 1.5))


def is_global(layer):
    return layer % 8 == 7


def read_safetensors(path, names=None):
    """Minimal safetensors reader -> {name: np.uint16 array} (BF16 bits)."""
    with open(path, "rb") as f:
        n = int.from_bytes(f.read(8), "little")
        header = json.loads(f.read(n))
    start = 8 + n
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    out = {}
    for name, t in header.items():
        if name == "__metadata__" or (names is not None and name not in names):
            continue
        a, b = t["data_offsets"]
        out[name] = np.frombuffer(mm[start + a:start + b], dtype=np.uint16).reshape(t["shape"])
    return out


class Weights:
    """FP32 copies of the BF16 weights of a model directory (all values are exact)."""

    def __init__(self, directory):
        raw = read_safetensors(os.path.join(directory, "model.safetensors"))
        t = lambda a: bf_t(torch.from_numpy(a.astype(np.int32)))
        self.embed_bits = raw["model.embed_tokens.weight"]
        self.head = t(raw["lm_head.weight"])
        self.final = torch.from_numpy(raw["model.norm.weight"].astype(np.int32))
        self.layers = []
        for i in range(LAYERS):
            p = f"model.layers.layers.{i}."
            g = lambda s: raw[p + s + ".weight"]
            self.layers.append(dict(
                qkv=t(g("mixer.qkv_proj")), o=t(g("mixer.o_proj")), up=t(g("mlp.gate_up_proj")),
                down=t(g("mlp.down_proj")),
                q_norm=torch.from_numpy(g("mixer.q_norm").astype(np.int32)),
                k_norm=torch.from_numpy(g("mixer.k_norm").astype(np.int32)),
                pre=torch.from_numpy(g("pre_mixer_norm").astype(np.int32)),
                post=torch.from_numpy(g("post_mixer_norm").astype(np.int32)),
                pre_mlp=torch.from_numpy(g("pre_mlp_norm").astype(np.int32)),
                post_mlp=torch.from_numpy(g("post_mlp_norm").astype(np.int32))))
        with open(os.path.join(directory, "config-mlx.json")) as f:
            freqs = json.load(f)["plamo_rope_inv_freq"]
        self.f_local, self.f_full = freqs["local"], freqs["full"]

    def embed(self, tokens):
        return bf_t(torch.from_numpy(self.embed_bits[np.asarray(tokens)].astype(np.int32)))


def gain(w_bits, offset):
    """roundbf(bf(w) + offset) (Kernels.metal:70)."""
    return roundbf_t(bf_t(w_bits) + torch.tensor(offset, dtype=torch.float32))


def norm(x, w_bits, offset):
    """Kernels.metal:59-72 (without residual): x [T, n] FP32."""
    n = x.shape[-1]
    r = 1.0 / torch.sqrt((x * x).sum(-1, keepdim=True) / n + torch.tensor(1e-6, dtype=torch.float32))
    return roundbf_t(roundbf_t(x * r) * gain(w_bits, offset))


def rotate(z, c, s):
    """rotated() (Kernels.metal:261-274): z [..., 128]; c, s [..., 64] broadcastable."""
    c2, s2 = torch.cat([c, c], -1), torch.cat([s, s], -1)
    other = torch.cat([-z[..., 64:], z[..., :64]], -1)
    return roundbf_t(roundbf_t(z * c2) + roundbf_t(other * s2))


class Oracle:
    """Runtime (Runtime.swift:128-553) on the CPU for one sequence.

    ``dots="fp32"`` (default) takes every dot product and sum (linear layers, norms,
    attention scores, softmax denominators, P.V) in torch's FP32 order and exp in torch FP32;
    ``dots="exact"`` computes each of them in FP64 and rounds once to FP32 (BF16 x BF16
    products are exact in FP64 and sums of at most 32768 terms carry ~2^-38 relative error,
    so each is the correctly rounded FP32 value; exp likewise).  The exact mode therefore
    gives the same bits on every machine, while torch's FP32 order changes with the host's
    thread count and vector width.  The two modes differ only in those roundings; the
    difference of their logits is the summation-order noise floor of the model
    (tests/test_noise_floor.py)."""

    def __init__(self, weights, context, local_capacity=None, dots="fp32"):
        assert dots in ("fp32", "exact")
        self.dots = dots
        self.w = weights
        self.context = context
        self.batch_limit = min(context, 16)
        cap_local = local_capacity or min(context, WINDOW + self.batch_limit)
        self.capacity = [context if is_global(i) else cap_local for i in range(LAYERS)]
        lc, ls = rope.local_table(weights.f_local, min(context, WINDOW + 16))
        gc, gs = rope.global_table(weights.f_full, context)
        self.local = (torch.from_numpy(lc), torch.from_numpy(ls))
        self.glob = (torch.from_numpy(gc), torch.from_numpy(gs))
        self.keys = [torch.zeros(c, HEAD_DIM, dtype=torch.int32) for c in self.capacity]
        self.values = [torch.zeros(c, HEAD_DIM, dtype=torch.int32) for c in self.capacity]
        self.reset()

    def reset(self):
        self.position = 0
        self.logit_bits = None
        self.logits_fp32 = None
        self.hidden = None

    def _mm(self, x, w):
        """x @ w.T with the dot products of the selected mode."""
        if self.dots == "fp32":
            return x @ w.T
        # FP64 copies are kept on the weights object, shared by every oracle over it
        cache = self.w.__dict__.setdefault("_w64", {})
        key = id(w)
        if key not in cache:
            cache[key] = (w, w.double())
        return (x.double() @ cache[key][1].T).float()

    # Reductions and exponentials of the selected mode: torch FP32, or FP64 rounded once to
    # FP32 (sums and exp), which no thread count, vector width or CPU changes.
    def _sum(self, t):
        if self.dots == "fp32":
            return t.sum(-1, keepdim=True)
        return t.double().sum(-1, keepdim=True).float()

    def _exp(self, t):
        if self.dots == "fp32":
            return torch.exp(t)
        return torch.exp(t.double()).float()

    def _einsum(self, eq, a, b):
        if self.dots == "fp32":
            return torch.einsum(eq, a, b)
        return torch.einsum(eq, a.double(), b.double()).float()

    def _norm(self, x, w_bits, offset):
        """``norm`` with this mode's sum of squares."""
        n = x.shape[-1]
        r = 1.0 / torch.sqrt(self._sum(x * x) / n + torch.tensor(1e-6, dtype=torch.float32))
        return roundbf_t(roundbf_t(x * r) * gain(w_bits, offset))

    def _softmax_pv(self, s, values):
        """softmax over the last axis of the scaled, masked scores, then roundbf(P.V)."""
        m = s.max(-1, keepdim=True).values
        e = self._exp(s - m)
        p = e / self._sum(e)
        return roundbf_t(self._einsum("thk,kd->thd", p, values))

    def _attention(self, layer, q_heads, T, p0):
        """Runtime.swift:389-444 for a chunk of T tokens starting at p0."""
        full, cap = is_global(layer), self.capacity[layer]
        base = 0 if full else max(0, p0 - (WINDOW - 1))
        count = p0 + T - base
        r = torch.arange(count)
        phys = (base + r) % cap
        keys = bf_t(self.keys[layer][phys])
        if not full:
            keys = rotate(keys, self.local[0][r], self.local[1][r])
        scores = self._einsum("thd,kd->thk", q_heads, keys)
        end = torch.arange(T) + p0 - base + 1
        begin = torch.zeros(T, dtype=torch.long) if full else torch.clamp(end - WINDOW, min=0)
        kk = torch.arange(count)[None, :]
        visible = (kk >= begin[:, None]) & (kk < end[:, None])
        s = torch.where(visible[:, None, :], scores * torch.tensor(SCALE), torch.tensor(-np.inf))
        values = bf_t(self.values[layer][phys])
        return self._softmax_pv(s, values).reshape(T, HEADS * HEAD_DIM)

    def forward(self, tokens, output=True):
        """Runtime.forward (Runtime.swift:327-467) for 1..16 tokens."""
        T, p0 = len(tokens), self.position
        if not (0 < T <= self.batch_limit) or any(not (0 <= t < VOCAB) for t in tokens) or \
                p0 + T > self.context:
            raise ValueError("Invalid tokens or context exhausted")
        x = self.w.embed(tokens)
        xn = self._norm(x, self.w.layers[0]["pre"], 1.0)
        pos = torch.arange(T) + p0
        for i, L in enumerate(self.w.layers):
            full, cap = is_global(i), self.capacity[i]
            base = 0 if full else max(0, p0 - (WINDOW - 1))
            qkv = roundbf_t(self._mm(xn, L["qkv"]))
            heads = qkv[:, :17 * HEAD_DIM].reshape(T, 17, HEAD_DIM)
            r = 1.0 / torch.sqrt(self._sum(heads * heads) / 128.0 + torch.tensor(1e-6))
            g = torch.cat([gain(L["q_norm"], 1.0)[None].expand(16, -1), gain(L["k_norm"], 1.0)[None]], 0)
            z = roundbf_t(roundbf_t(heads * r) * g)
            if full:
                cq, sq = self.glob[0][pos], self.glob[1][pos]
            else:
                cq, sq = self.local[0][pos - base], self.local[1][pos - base]
            q = rotate(z[:, :16], cq[:, None], sq[:, None])
            k = rotate(z[:, 16], self.glob[0][pos], self.glob[1][pos]) if full else z[:, 16]
            self.keys[i][pos % cap] = bits_t(k)
            self.values[i][pos % cap] = bits_t(qkv[:, 17 * HEAD_DIM:])
            att = self._attention(i, q, T, p0)
            o = roundbf_t(self._mm(att, L["o"]))
            x = roundbf_t(x + self._norm(o, L["post"], 0.2))
            xn = self._norm(x, L["pre_mlp"], 1.0)
            gu = roundbf_t(self._mm(xn, L["up"]))
            gate = gu[:, :INTER]
            act = roundbf_t(roundbf_t(gate / (1.0 + self._exp(-gate))) * gu[:, INTER:])
            d = roundbf_t(self._mm(act, L["down"]))
            x = roundbf_t(x + self._norm(d, L["post_mlp"], POST_MLP_OFFSET))
            if i + 1 < LAYERS:
                xn = self._norm(x, self.w.layers[i + 1]["pre"], 1.0)
        self.position += T
        if not output:
            return -1
        h = self._norm(x[-1:], self.w.final, 1.0)
        self.hidden = h[0]
        self.logits_fp32 = self._mm(h, self.w.head)[0]
        self.logit_bits = bits_t(self.logits_fp32)
        from .sampler import argmax_gpu
        return argmax_gpu(bf_t(self.logit_bits).numpy())

    def prefill(self, tokens):
        """Runtime.prefill/fill (Runtime.swift:473-483): 16-token chunks, output on the last."""
        if not tokens or self.position + len(tokens) > self.context:
            raise ValueError("Input exceeds context")
        nxt = -1
        for s in range(0, len(tokens), self.batch_limit):
            e = min(s + self.batch_limit, len(tokens))
            nxt = self.forward(list(tokens[s:e]), output=e == len(tokens))
        return nxt

    def fill(self, tokens):
        """``prefill`` computed a prompt at a time (long prompts).  The linear layers, norms
        and SwiGLU act on each row independently, so they run over every prompt row at once;
        each row's query and key coordinates follow its 16-token chunk's RoPE base
        (Runtime.swift:389-399, chunks counted from the current position, as ``prefill``);
        attention sees each query's visible keys, [pos-2047, pos] on local layers and
        [0, pos] on global ones.  Every key of the prompt is written before attention, so the
        prompt and the window before it must fit the ring without overwriting."""
        T, p0 = len(tokens), self.position
        if not tokens or p0 + T > self.context or any(not (0 <= t < VOCAB) for t in tokens):
            raise ValueError("Input exceeds context")
        if p0 + T > max(0, p0 - (WINDOW - 1)) + min(self.capacity):
            raise ValueError("prompt does not fit the ring at once")
        x = self.w.embed(tokens)
        xn = self._norm(x, self.w.layers[0]["pre"], 1.0)
        pos = torch.arange(T) + p0
        chunk_base = torch.clamp(p0 + (torch.arange(T) // self.batch_limit) * self.batch_limit - (WINDOW - 1), min=0)
        for i, L in enumerate(self.w.layers):
            full, cap = is_global(i), self.capacity[i]
            qkv = roundbf_t(self._mm(xn, L["qkv"]))
            heads = qkv[:, :17 * HEAD_DIM].reshape(T, 17, HEAD_DIM)
            r = 1.0 / torch.sqrt(self._sum(heads * heads) / 128.0 + torch.tensor(1e-6))
            g = torch.cat([gain(L["q_norm"], 1.0)[None].expand(16, -1), gain(L["k_norm"], 1.0)[None]], 0)
            z = roundbf_t(roundbf_t(heads * r) * g)
            if full:
                cq, sq = self.glob[0][pos], self.glob[1][pos]
            else:
                cq, sq = self.local[0][pos - chunk_base], self.local[1][pos - chunk_base]
            q = rotate(z[:, :16], cq[:, None], sq[:, None])
            k = rotate(z[:, 16], self.glob[0][pos], self.glob[1][pos]) if full else z[:, 16]
            self.keys[i][pos % cap] = bits_t(k)
            self.values[i][pos % cap] = bits_t(qkv[:, 17 * HEAD_DIM:])
            att = torch.empty(T, HEADS * HEAD_DIM)
            bases = [0] if full else sorted(set(chunk_base.tolist()))
            for b in bases:
                rows = torch.arange(T) if full else torch.nonzero(chunk_base == b)[:, 0]
                att[rows] = self._attend_rows(i, q[rows], pos[rows], b)
            o = roundbf_t(self._mm(att, L["o"]))
            x = roundbf_t(x + self._norm(o, L["post"], 0.2))
            xn = self._norm(x, L["pre_mlp"], 1.0)
            gu = roundbf_t(self._mm(xn, L["up"]))
            gate = gu[:, :INTER]
            act = roundbf_t(roundbf_t(gate / (1.0 + self._exp(-gate))) * gu[:, INTER:])
            d = roundbf_t(self._mm(act, L["down"]))
            x = roundbf_t(x + self._norm(d, L["post_mlp"], POST_MLP_OFFSET))
            if i + 1 < LAYERS:
                xn = self._norm(x, self.w.layers[i + 1]["pre"], 1.0)
        self.position += T
        h = self._norm(x[-1:], self.w.final, 1.0)
        self.hidden = h[0]
        self.logits_fp32 = self._mm(h, self.w.head)[0]
        self.logit_bits = bits_t(self.logits_fp32)
        from .sampler import argmax_gpu
        return argmax_gpu(bf_t(self.logit_bits).numpy())

    def _attend_rows(self, layer, q, pos, base, block=256):
        """Attention of queries q [G, 16, 128] at positions `pos` whose keys rotate with RoPE
        base `base` (local layers; 0 and unused on global ones), in the softmax/attend
        arithmetic of ``_attention``."""
        full, cap = is_global(layer), self.capacity[layer]
        last = int(pos.max())
        r = torch.arange(last + 1 - base)
        phys = (base + r) % cap
        keys = bf_t(self.keys[layer][phys])
        if not full:
            keys = rotate(keys, self.local[0][r], self.local[1][r])
        values = bf_t(self.values[layer][phys])
        kabs = base + r
        out = torch.empty(q.shape[0], HEADS * HEAD_DIM)
        for s in range(0, q.shape[0], block):
            qq, pp = q[s:s + block], pos[s:s + block]
            scores = self._einsum("thd,kd->thk", qq, keys)
            lo = torch.zeros_like(pp) if full else torch.clamp(pp - (WINDOW - 1), min=0)
            visible = (kabs[None, :] >= lo[:, None]) & (kabs[None, :] <= pp[:, None])
            sc = torch.where(visible[:, None, :], scores * torch.tensor(SCALE), torch.tensor(-np.inf))
            out[s:s + block] = self._softmax_pv(sc, values).reshape(-1, HEADS * HEAD_DIM)
        return out

    def logits(self):
        """Runtime.logits(into:) (Runtime.swift:547-552): BF16 logits widened to FP32."""
        return bf_t(self.logit_bits).numpy()


def greedy(oracle, prompt, max_tokens, sampling=None):
    """The token loop of Main.swift:235-288 -> (generated ids, stop reason).
    ``sampling`` = dict(penalty, frequency, ngram) applies Sampler.select over generated-only
    history (Main.swift:237-244)."""
    from .sampler import select
    oracle.reset()
    generated = []

    def sample(greedy_id):
        if not sampling:
            return greedy_id
        return select(oracle.logits().copy(), generated, sampling.get("penalty", 1.0),
                      sampling.get("ngram", 0), sampling.get("frequency", 0.0))

    nxt = sample(oracle.prefill(prompt))
    for i in range(max_tokens):
        if nxt in (1, 16):
            return generated, "stop"
        generated.append(nxt)
        if i + 1 < max_tokens:
            nxt = sample(oracle.forward([nxt]))
    return generated, None


def textbook_logits(weights, tokens):
    """Independent FP32 forward written from the HF/MLX layer algorithm
    (scripts/verify_long.py:24-56; norm/rope from scripts/auxiliary.py:35-47) for a prompt of
    at most 2048 tokens processed at once: standard RMSNorm with the stored-offset gains,
    rotate-half RoPE (global: mscale 1.5545177444479562; local: none) at absolute positions,
    causal (global) or 2048-window causal (local) attention, SwiGLU, untied LM head.
    No intermediate BF16 rounding.  Returns FP32 logits of the last position."""
    T = len(tokens)
    assert T <= WINDOW
    x = weights.embed(tokens).double()

    def rms(v, w_bits, offset):
        g = (bf_t(w_bits).double() + offset)
        return v / torch.sqrt((v * v).mean(-1, keepdim=True) + 1e-6) * g

    pos = torch.arange(T, dtype=torch.float64)

    def rope_apply(v, freqs, mscale):
        f = torch.tensor(freqs, dtype=torch.float64)
        ang = pos[:, None] * f[None, :]
        c = torch.cat([torch.cos(ang), torch.cos(ang)], -1) * mscale
        s = torch.cat([torch.sin(ang), torch.sin(ang)], -1) * mscale
        other = torch.cat([-v[..., 64:], v[..., :64]], -1)
        return v * c[:, None, :] + other * s[:, None, :]

    for i, L in enumerate(weights.layers):
        h = rms(x, L["pre"], 1.0)
        qkv = h @ L["qkv"].double().T
        q = qkv[:, :2048].reshape(T, 16, 128)
        k = qkv[:, 2048:2176].reshape(T, 1, 128)
        v = qkv[:, 2176:]
        q = rms(q, L["q_norm"], 1.0)
        k = rms(k, L["k_norm"], 1.0)
        if is_global(i):
            q, k = rope_apply(q, weights.f_full, 1.5545177444479562), rope_apply(k, weights.f_full, 1.5545177444479562)
        else:
            q, k = rope_apply(q, weights.f_local, 1.0), rope_apply(k, weights.f_local, 1.0)
        scores = torch.einsum("thd,sd->ths", q, k[:, 0]) * (128 ** -0.5)
        qp, kp = torch.arange(T)[:, None], torch.arange(T)[None, :]
        mask = kp <= qp
        if not is_global(i):
            mask = mask & (kp > qp - WINDOW)
        scores = scores.masked_fill(~mask[:, None, :], -np.inf)
        att = torch.einsum("ths,sd->thd", torch.softmax(scores, -1), v).reshape(T, 2048)
        x = x + rms(att @ L["o"].double().T, L["post"], 0.2)
        h = rms(x, L["pre_mlp"], 1.0)
        gu = h @ L["up"].double().T
        a = torch.nn.functional.silu(gu[:, :INTER]) * gu[:, INTER:]
        x = x + rms(a @ L["down"].double().T, L["post_mlp"], POST_MLP_OFFSET)
    h = rms(x[-1:], weights.final, 1.0)
    return (h @ weights.head.double().T)[0].float()
