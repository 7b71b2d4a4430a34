"""Bit-exact prefill: the MFMA prefill kernels and the whole GPU prefill equal the order-exact
CPU restatement (oracle/exact_prefill.py) in every bit.

* plamo_kernel_gemm at the four projection shapes (raw FP32 accumulators, BF16 outputs, the
  gate_up SwiGLU epilogue), plain and .p12 weights, ragged token counts;
* plamo_kernel_attention_prefill on local and global layers, chunk bases, a wrapped ring,
  and key ranges split over two and three parts;
* Runtime.prefill of the config-1 prompt (Runtime.swift:469-483): logits, final hidden row,
  next token and every layer's K/V, plain and .p12 weights; then decode steps on the
  prefilled state, against the decode twin on the twin's prefilled state.
"""
import numpy as np
import pytest
import torch

import plamo_hip
from oracle import exact, exact_prefill as xp, p12, rope
from oracle.bf16 import bf_np, bits_np, roundbf_np
from plamo_hip import native

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def ptr(t):
    return t.data_ptr() if t is not None else 0


@pytest.fixture(scope="module")
def lib():
    return native.load()


def _gemm(lib, w, x, mode, packed):
    m, n = w.shape
    tokens = x.shape[0]
    if packed:
        data, offsets, minima = p12.pack(w)
        wd, td = dev(data), dev(p12.tag(offsets, minima).view(np.int32))
    else:
        wd, td = dev(w.view(np.int16)), None
    xd = dev(x.view(np.int16))
    cols = 6144 if mode == 3 else m
    y = torch.empty(tokens * cols, dtype=torch.float32 if mode == 2 else torch.int16, device="cuda")
    assert lib.plamo_kernel_gemm(ptr(wd), ptr(td), ptr(xd), ptr(y), n, m, tokens, mode, 0) == 0
    torch.cuda.synchronize()
    out = y.cpu().numpy().reshape(tokens, cols)
    return out if mode == 2 else out.view(np.uint16)


@pytest.mark.parametrize("name,m,n,tokens", [("qkv", 2304, 1536, 130), ("o", 1536, 2048, 77),
                                             ("gate_up", 12288, 1536, 40), ("down", 1536, 6144, 57)])
def test_gemm_bit_exact(lib, name, m, n, tokens):
    print(f"  gemm {name} {m}x{n} tokens={tokens}", flush=True)
    rng = np.random.default_rng(m + n + tokens)
    w = bits_np(rng.standard_normal((m, n)).astype(np.float32) * 0.02)
    x = bits_np(rng.standard_normal((tokens, n)).astype(np.float32))
    want = xp.mfma_gemm(w, x)
    for packed in (False, True):
        raw = _gemm(lib, w, x, 2, packed)
        bad = int(np.sum(raw.view(np.uint32) != want.view(np.uint32)))
        assert bad == 0, (name, packed, bad)
        if name == "gate_up":
            g, u = roundbf_np(want[:, :6144]), roundbf_np(want[:, 6144:])
            act = bits_np(roundbf_np(g / (np.float32(1) + exact.exp_det(-g))) * u)
            assert np.array_equal(_gemm(lib, w, x, 3, packed), act), packed
        else:
            assert np.array_equal(_gemm(lib, w, x, 1, packed), bits_np(want)), packed


@pytest.mark.parametrize("p0,tokens,cap,full", [
    (0, 100, 2064, False),     # ragged token count, keys from position 0, two tiles
    (2040, 24, 2080, False),   # chunk bases 0 and 9 in one call
    (3000, 40, 2112, False),   # chunk-relative coordinates and a wrapped ring
    (0, 64, 64, True),         # global, keys exactly the tokens
    (500, 37, 600, True),      # global, key tiles split over two parts
    (1100, 50, 1200, True),    # global, three parts merged
])
def test_flash_bit_exact(lib, p0, tokens, cap, full):
    print(f"  flash p0={p0} tokens={tokens} cap={cap} full={full}", flush=True)
    rng = np.random.default_rng(p0 + tokens)
    q = bits_np(rng.standard_normal((tokens, 16, 128)).astype(np.float32))
    keys = bits_np(rng.standard_normal((cap, 128)).astype(np.float32))
    values = bits_np(rng.standard_normal((cap, 128)).astype(np.float32))
    freqs = (10000.0 ** (-np.arange(64, dtype=np.float64) / 64)).astype(np.float32)
    c, s = rope.local_table(freqs, rope.LOCAL_ROWS)
    packed = bits_np(c).astype(np.uint32) | (bits_np(s).astype(np.uint32) << 16)
    out = torch.full((tokens, 2048), -1, dtype=torch.int16, device="cuda")
    # device copies held until the kernel has run
    qd, kd, vd, rd = (dev(a) for a in (q.view(np.int16), keys.view(np.int16), values.view(np.int16),
                                        packed.view(np.int32)))
    rc = lib.plamo_kernel_attention_prefill(ptr(qd), ptr(kd), ptr(vd), cap, p0, tokens, 1 if full else 0, ptr(rd),
                                            ptr(out), 0)
    assert rc == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    want = xp.flash(q, keys, values, bits_np(c), bits_np(s), cap, p0, full)
    bad = int(np.sum(got != want))
    assert bad == 0, (bad, got.size)


@pytest.fixture(scope="module")
def twin_prefill(oracle_weights, golden):
    """The twin's config-1 prefill on a 96-position context (local ring min(96, 2048 + 96))."""
    prompt = golden["config1"]["prompt"]
    ex = exact.ExactDecoder(oracle_weights, 96, 96)
    out = xp.ExactPrefill(ex).prefill(prompt)
    return prompt, ex, out


@pytest.mark.parametrize("packed", [False, True])
def test_prefill_bit_exact(model_dir, twin_prefill, packed):
    d, sha = model_dir
    prompt, ex, (bits, hidden, nxt) = twin_prefill
    rt = plamo_hip.Runtime(d, 96, packed=packed, source_sha256=sha)
    assert rt.stats()["local_capacity"] == ex.cap[0]
    got = rt.prefill(prompt)
    print(f"  prefill {len(prompt)} tokens packed={packed}: next {got} (twin {nxt})", flush=True)
    assert np.array_equal(rt.logit_bits(), bits)
    assert np.array_equal(rt.hidden().view(np.uint32), hidden.view(np.uint32))
    assert got == nxt
    n = len(prompt)
    for layer in range(16):
        k, v = rt.kv(layer)
        assert np.array_equal(k[:n], ex.keys[layer][:n]), layer
        assert np.array_equal(v[:n], ex.values[layer][:n]), layer
    rt.close()


def test_config3_prefill_first_layers_bit_exact(model_dir, oracle_weights, golden):
    # configs[2] itself: the 2048-token prompt in one chunk.  The twin runs layer 0 in full
    # (qkv, flash attention over the 2048-key causal window, o, norms, gate_up, down) and
    # layer 1 up to its KV write; every key and value of both layers equals the GPU's.
    g = golden["config3"]
    prompt = np.random.default_rng(g["prompt_seed"]).integers(1024, 107520, g["length"]).tolist()
    d, _ = model_dir
    rt = plamo_hip.Runtime(d, 2048)
    try:
        rt.prefill(prompt)
        kv = [rt.kv(layer) for layer in (0, 1)]
        cap = rt.stats()["local_capacity"]
    finally:
        rt.close()
    ex = exact.ExactDecoder(oracle_weights, 2048, cap)
    xp.ExactPrefill(ex).prefill(prompt, kv_layers=2)
    n = len(prompt)
    for layer, (k, v) in zip((0, 1), kv):
        bad_k = int(np.sum(k[:n] != ex.keys[layer][:n]))
        bad_v = int(np.sum(v[:n] != ex.values[layer][:n]))
        print(f"  config3 layer {layer}: {bad_k} key / {bad_v} value words differ", flush=True)
        assert bad_k == 0 and bad_v == 0, layer


def test_config3_prefill_all_layers_match_twin_digests(model_dir, golden):
    # configs[2] through all 16 layers and the head.  The full twin runs for minutes, so
    # tests/golden/make_config3_digest.py ran it on the CPU and kept SHA-256 digests of its
    # keys, values, logits and hidden row; the GPU prefill's bytes must hash to the same.
    import hashlib
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", "config3_prefill_digest.json")) as f:
        want = json.load(f)
    d, sha = model_dir
    assert want["model_sha256"] == sha
    g = golden["config3"]
    prompt = np.random.default_rng(g["prompt_seed"]).integers(1024, 107520, g["length"]).tolist()
    n = len(prompt)
    assert n == want["prompt_tokens"]

    def digest(a, dtype):
        return hashlib.sha256(np.ascontiguousarray(a, dtype=dtype).tobytes()).hexdigest()

    rt = plamo_hip.Runtime(d, want["context"], source_sha256=sha)
    try:
        nxt = rt.prefill(prompt)
        bad = []
        for layer in range(16):
            k, v = rt.kv(layer)
            for name, a in (("keys", k[:n]), ("values", v[:n])):
                if digest(a, np.uint16) != want["layers"][layer][name]:
                    bad.append(f"layer {layer} {name}")
        if digest(rt.logit_bits(), np.uint16) != want["logits"]:
            bad.append("logits")
        if digest(rt.hidden().view(np.uint32), np.uint32) != want["hidden"]:
            bad.append("hidden")
    finally:
        rt.close()
    print(f"  config3 full prefill: next {nxt} (twin {want['next']}), differing: {bad or 'none'}", flush=True)
    assert not bad, bad
    assert nxt == want["next"]


def test_decode_after_prefill_bit_exact(model_dir, oracle_weights, twin_prefill):
    # greedy decode on the prefilled KV: the GPU step equals the decode twin run on the
    # prefill twin's KV, step after step
    d, _ = model_dir
    prompt, ex0, (_, _, nxt) = twin_prefill
    ex = exact.ExactDecoder(oracle_weights, 96, 96)
    ex.keys = [k.copy() for k in ex0.keys]
    ex.values = [v.copy() for v in ex0.values]
    rt = plamo_hip.Runtime(d, 96)
    assert rt.prefill(prompt) == nxt
    t = nxt
    for pos in range(len(prompt), len(prompt) + 12):
        got = rt.forward([t])
        bits, hidden, want = ex.step(t, pos)
        assert np.array_equal(rt.logit_bits(), bits), pos
        assert got == want, pos
        t = got
    rt.close()
