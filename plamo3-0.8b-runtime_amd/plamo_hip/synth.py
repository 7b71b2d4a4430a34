"""Random-init PLaMo-3 0.8B-shaped model directories (synthetic data for tests and benches).

A model directory holds what ``Runtime.init`` reads (Runtime.swift:180-192,268-274):

* ``config.json``      -- the configuration the loader insists on (Runtime.swift:181-188).
* ``config-mlx.json``  -- ``plamo_rope_inv_freq.local/full`` (64 values each), here the
  textbook inverse frequencies ``1/theta**(i/64)`` for theta 1e4 (local) and 1e6 (full).
* ``model.safetensors``-- BF16 tensors under the reference's names and shapes
  (Runtime.swift:59-62,233-246).

Weights are N(0, 0.02) drawn with ``numpy.random.default_rng(seed)`` in the canonical order
(embedding; per layer qkv, o, gate_up, down; lm_head), FP32 -> BF16 round-to-nearest-even.
Norm tensors store ``1 - offset`` so every effective gain ``roundbf(bf(w) + offset)`` is 1.0:
0.0 for the +1.0 norms (pre-mixer, pre-MLP, final, q, k), 0.8 for post-mixer (offset 0.2)
and 0.9105573 for post-MLP (offset 5^-1.5) (offsets: Runtime.swift:377,446,450-451,455).
"""
import hashlib
import json
import os
import struct

import numpy as np

HIDDEN, HEAD_DIM, INTER, VOCAB, LAYERS = 1536, 128, 6144, 107520, 16

CONFIG = {
    "model_type": "plamo3", "dtype": "bfloat16", "hidden_size": 1536, "num_hidden_layers": 16,
    "num_attention_heads": 16, "num_key_value_heads": 1, "head_dim": 128,
    "intermediate_size": 6144, "vocab_size": 107520, "window_size": 2048,
    "sliding_window_pattern": 8, "tie_word_embeddings": False, "scale_embedding": False,
    "rope_theta": 1000000.0, "rope_local_theta": 10000.0, "rope_scaling_factor": 256.0,
    "rms_norm_eps": 1e-06,
}


def _bf16(a):
    u = a.view(np.uint32)
    r = (u >> 16) & 1
    r += 0x7FFF
    r += u
    r >>= 16
    return r.astype(np.uint16)


def tensor_plan():
    """[(name, shape, kind)] in file order; kind is 'random' or a stored norm value."""
    plan = [("model.embed_tokens.weight", (VOCAB, HIDDEN), "random")]
    for i in range(LAYERS):
        p = f"model.layers.layers.{i}."
        plan += [(p + "mixer.qkv_proj.weight", (2304, HIDDEN), "random"),
                 (p + "mixer.o_proj.weight", (HIDDEN, 2048), "random"),
                 (p + "mixer.q_norm.weight", (HEAD_DIM,), 0.0),
                 (p + "mixer.k_norm.weight", (HEAD_DIM,), 0.0),
                 (p + "mlp.gate_up_proj.weight", (2 * INTER, HIDDEN), "random"),
                 (p + "mlp.down_proj.weight", (HIDDEN, INTER), "random"),
                 (p + "pre_mixer_norm.weight", (HIDDEN,), 0.0),
                 (p + "post_mixer_norm.weight", (HIDDEN,), 0.8),
                 (p + "pre_mlp_norm.weight", (HIDDEN,), 0.0),
                 (p + "post_mlp_norm.weight", (HIDDEN,), 0.9105573)]
    plan += [("model.norm.weight", (HIDDEN,), 0.0), ("lm_head.weight", (VOCAB, HIDDEN), "random")]
    return plan


def frequencies():
    i = np.arange(64, dtype=np.float64)
    return (1.0 / (10000.0 ** (i / 64.0))).tolist(), (1.0 / (1000000.0 ** (i / 64.0))).tolist()


def write_model(directory, seed=0, std=0.02):
    """Write a complete synthetic model directory; returns the safetensors SHA-256."""
    os.makedirs(directory, exist_ok=True)
    plan = tensor_plan()
    header, offset = {}, 0
    for name, shape, _ in plan:
        size = int(np.prod(shape)) * 2
        header[name] = {"dtype": "BF16", "shape": list(shape), "data_offsets": [offset, offset + size]}
        offset += size
    header["__metadata__"] = {"format": "pt", "generator": f"plamo_hip.synth seed={seed} std={std}"}
    blob = json.dumps(header, separators=(",", ":")).encode()
    blob += b" " * ((-(8 + len(blob))) % 64)
    path = os.path.join(directory, "model.safetensors")
    part = path + ".part"
    rng = np.random.default_rng(seed)
    digest = hashlib.sha256()
    chunk = 1 << 22
    with open(part, "wb") as f:
        head = struct.pack("<Q", len(blob)) + blob
        f.write(head)
        digest.update(head)
        for name, shape, kind in plan:
            n = int(np.prod(shape))
            if kind == "random":
                for s in range(0, n, chunk):
                    a = rng.standard_normal(min(chunk, n - s), dtype=np.float32)
                    a *= np.float32(std)
                    b = _bf16(a).tobytes()
                    f.write(b)
                    digest.update(b)
            else:
                b = _bf16(np.full(n, kind, dtype=np.float32)).tobytes()
                f.write(b)
                digest.update(b)
    os.replace(part, path)
    local, full = frequencies()
    with open(os.path.join(directory, "config.json"), "w") as f:
        json.dump(CONFIG, f, indent=1)
    with open(os.path.join(directory, "config-mlx.json"), "w") as f:
        json.dump({"plamo_rope_inv_freq": {"local": local, "full": full}}, f)
    sha = digest.hexdigest()
    with open(os.path.join(directory, "model.sha256"), "w") as f:
        f.write(sha + "\n")
    return sha


def aux_plan():
    """[(name, shape, kind)] of auxiliary.safetensors (Auxiliary.swift:72-111): the QSA indexers
    of the two global layers and the MTP head."""
    plan = []
    for layer in (7, 15):
        p = f"qsa.{layer}."
        plan += [(p + "proj.weight", (640, HIDDEN), "random"), (p + "q_norm.weight", (HEAD_DIM,), 0.0),
                 (p + "k_norm.weight", (HEAD_DIM,), 0.0)]
    plan += [("mtp.heads.0.up.weight", (256, 2 * HIDDEN), "random"),
             ("mtp.heads.0.down.weight", (HIDDEN, 256), "random")]
    return plan


def write_auxiliary(directory, teacher_sha256, seed=100, std=0.02):
    """Random-init adapters in the plamo-aux-v1 layout the loader checks (Auxiliary.swift:29-40;
    header padded to 64 bytes as scripts/auxiliary.py:12-31 writes it), trained against the
    model whose safetensors SHA-256 is `teacher_sha256`."""
    plan = aux_plan()
    header, offset = {}, 0
    for name, shape, _ in plan:
        size = int(np.prod(shape)) * 2
        header[name] = {"dtype": "BF16", "shape": list(shape), "data_offsets": [offset, offset + size]}
        offset += size
    header["__metadata__"] = {"format": "plamo-aux-v1", "teacher_sha256": teacher_sha256, "rank": "256",
                              "qsa_steps": "1", "mtp_steps": "1"}
    blob = json.dumps(header, separators=(",", ":")).encode()
    blob += b" " * ((-(8 + len(blob))) % 64)
    rng = np.random.default_rng(seed)
    path = os.path.join(directory, "auxiliary.safetensors")
    with open(path + ".part", "wb") as f:
        f.write(struct.pack("<Q", len(blob)) + blob)
        for name, shape, kind in plan:
            n = int(np.prod(shape))
            a = (rng.standard_normal(n, dtype=np.float32) * np.float32(std)) if kind == "random" else \
                np.full(n, kind, dtype=np.float32)
            f.write(_bf16(a).tobytes())
    os.replace(path + ".part", path)
    return path


def ensure_model(directory=None, seed=0, packed=True):
    """Create (once) and return a synthetic model directory with model.p12 packed by the
    native packer.  Directory defaults to $PLAMO_MODEL_DIR or <tmp>/plamo_synth_seed<seed>."""
    import tempfile
    directory = directory or os.environ.get("PLAMO_MODEL_DIR") or \
        os.path.join(tempfile.gettempdir(), f"plamo_synth_seed{seed}")
    sha_path = os.path.join(directory, "model.sha256")
    if not os.path.exists(sha_path) or not os.path.exists(os.path.join(directory, "config-mlx.json")):
        write_model(directory, seed)
    sha = open(sha_path).read().strip()
    if not os.path.exists(os.path.join(directory, "auxiliary.safetensors")):
        write_auxiliary(directory, sha)
    if packed and not os.path.exists(os.path.join(directory, "model.p12")):
        from . import native
        native.pack(os.path.join(directory, "model.safetensors"), os.path.join(directory, "model.p12"), sha)
    return directory, sha


def tokenizer_records(seed=0):
    """A synthetic tokenizer.jsonl with the original's shape (Tokenizer.swift:90-95): 107,520
    entries, <|plamo:bos|> at 1 and <|plamo:tag|> at 16, BYTE tokens <0x80>..<0xFF> at 128-255
    and <0x00>..<0x7F> at 384-511, scored pieces of up to three characters over a small mixed
    alphabet, and single private-use characters filling the rest."""
    import random
    rng = random.Random(seed)
    n = 107520
    recs = [None] * n
    controls = ["<unk>", "<|plamo:bos|>", "<|plamo:eos|>", "<|plamo:pad|>"] + \
        [f"<|plamo:c{k}|>" for k in range(4, 16)] + ["<|plamo:tag|>", "<|plamo:msg|>", "<|plamo:key|>",
                                                    "<|plamo:val|>"]
    for i, p in enumerate(controls):
        recs[i] = [p, 0.0, "CONTROL"]
    for b in range(256):
        recs[b if b >= 128 else 384 + b] = [f"<0x{b:02X}>", 0.0, "BYTE"]
    alphabet = "abcdefgh ijk日本語の翻訳です。é,.\n"
    pieces = list(alphabet) + [a + b for a in alphabet for b in alphabet]
    pieces += [a + b + c for a in alphabet[:12] for b in alphabet[:12] for c in alphabet[:12]]
    free = iter(i for i in range(n) if recs[i] is None)
    for p in pieces:
        recs[next(free)] = [p, round(rng.uniform(-15, -1), 4), "NORMAL"]
    k = 0
    for i in free:
        recs[i] = [chr(0xF0000 + k), -30.0, "NORMAL"]
        k += 1
    return recs, alphabet


def ensure_tokenizer(directory=None, seed=0):
    """Writes the synthetic tokenizer.jsonl once; returns (path, alphabet)."""
    import tempfile
    directory = directory or os.path.join(tempfile.gettempdir(), "plamo_synth_tokenizer")
    os.makedirs(directory, exist_ok=True)
    path = os.path.join(directory, f"tokenizer-seed{seed}.jsonl")
    recs, alphabet = tokenizer_records(seed)
    if not os.path.exists(path):
        tmp = path + ".tmp"
        with open(tmp, "w", encoding="utf-8") as f:
            for r in recs:
                f.write(json.dumps(r, ensure_ascii=False) + "\n")
        os.replace(tmp, path)
    return path, alphabet
