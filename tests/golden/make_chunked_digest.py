"""Digests of the order-exact prefill twin over several 2048-token chunks:
tests/golden/chunked_prefill_digest.json.

Runtime.prefill runs a prompt in chunks (Runtime.swift:469-483); this runtime's chunks are
2048 tokens and its local rings hold min(context, 2048 + 2048) slots.  The default case is a
4,200-token prompt (numpy default_rng(12), ids 1024 .. 107519) at context 4,400: three
chunks (2048, 2048, 104 tokens), RoPE chunk bases above 0 from position 2048 on
(Runtime.swift:389-399), and a third chunk whose keys wrap the 4,096-slot local rings
(positions 4096.. go to slots 0..) while its queries attend over the wrapped window.  The
twin (oracle/exact_prefill.py) prefills it on the synthetic seed-0 model, all 16 layers,
then the last token's head.  That takes about half an hour of CPU, so the script records
SHA-256 digests and the GPU test compares the device prefill's bytes with them:

  layers[i].keys / values   the cached rows of layer i (BF16 bits, uint16 little-endian):
                            slots 0 .. min(n, capacity) - 1, i.e. every slot of a wrapped
                            local ring and rows 0 .. n-1 of a global layer;
  logits                    the last token's logits as the runtime returns them (BF16 bits);
  hidden                    the last token's final hidden row (FP32 bits);
  next                      the greedy next token.

    python tests/golden/make_chunked_digest.py [--tokens N --context C --seed S] [OUT]
    # from the repository root, CPU only; the defaults write the committed file
    # (configs[4]'s 30,720-token prompt is --tokens 30720 --context 32768 --seed 5: hours)
"""
import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
OUT = os.path.join(ROOT, "tests", "golden", "chunked_prefill_digest.json")
CHUNK = 2048
WINDOW = 2048


def sha(a, dtype):
    return hashlib.sha256(np.ascontiguousarray(a, dtype=dtype).tobytes()).hexdigest()


def prompt(seed, n):
    return np.random.default_rng(seed).integers(1024, 107520, n).tolist()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--tokens", type=int, default=4200)
    ap.add_argument("--context", type=int, default=4400)
    ap.add_argument("--seed", type=int, default=12)
    ap.add_argument("out", nargs="?", default=OUT)
    a = ap.parse_args()
    sys.path[:0] = [ROOT, os.path.join(ROOT, "plamo3-0.8b-runtime_amd")]
    from oracle import exact, exact_prefill as xp
    from oracle.model import Weights
    from plamo_hip import synth
    d, model_sha = synth.ensure_model(packed=True)
    toks = prompt(a.seed, a.tokens)
    n = len(toks)
    local = min(a.context, WINDOW + CHUNK)   # the runtime's ring rule
    ex = exact.ExactDecoder(Weights(d), a.context, local)
    t0 = time.time()
    bits, hidden, nxt = xp.ExactPrefill(ex).prefill(toks)
    print(f"twin prefill of {n} tokens: {time.time() - t0:.0f} s, next {nxt}", flush=True)
    out = {
        "prompt_tokens": n, "prompt_seed": a.seed, "context": a.context, "model_sha256": model_sha,
        "local_capacity": local,
        "layers": [{"keys": sha(ex.keys[i][:min(n, ex.cap[i])], np.uint16),
                    "values": sha(ex.values[i][:min(n, ex.cap[i])], np.uint16)} for i in range(16)],
        "logits": sha(bits, np.uint16), "hidden": sha(np.asarray(hidden, np.float32).view(np.uint32), np.uint32),
        "next": int(nxt),
    }
    with open(a.out, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print("wrote", a.out, flush=True)


if __name__ == "__main__":
    main()
