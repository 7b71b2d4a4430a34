"""Digests of the order-exact prefill twin on configs[2]: tests/golden/config3_prefill_digest.json.

The 2048-token configs[2] prompt (prompt_seed and length from tests/golden/manifest.json) is
prefilled in one chunk by oracle/exact_prefill.py on the synthetic seed-0 model at context
2048, all 16 layers, then the last token's head.  The full twin takes minutes of CPU (about
70 G multiply-adds through the MFMA accumulation model), too long for a test, so this script
records SHA-256 digests of what it produces and the GPU test compares the device prefill's
bytes with them:

  layers[i].keys / values   the n = 2048 cached key and value rows of layer i (BF16 bits,
                            ring slots 0 .. n-1, uint16 little-endian);
  logits                    the last token's logits as the runtime returns them (BF16 bits);
  hidden                    the last token's final hidden row (FP32 bits);
  next                      the greedy next token.

    python tests/golden/make_config3_digest.py [OUT]   # from the repository root, CPU only
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
OUT = os.path.join(ROOT, "tests", "golden", "config3_prefill_digest.json")
CONTEXT = 2048


def sha(a, dtype):
    return hashlib.sha256(np.ascontiguousarray(a, dtype=dtype).tobytes()).hexdigest()


def prompt(manifest):
    g = manifest["config3"]
    return np.random.default_rng(g["prompt_seed"]).integers(1024, 107520, g["length"]).tolist()


def main():
    sys.path[:0] = [ROOT, os.path.join(ROOT, "plamo3-0.8b-runtime_amd")]
    from oracle import exact, exact_prefill as xp
    from oracle.model import Weights
    from plamo_hip import synth
    with open(os.path.join(ROOT, "tests", "golden", "manifest.json")) as f:
        manifest = json.load(f)
    d, model_sha = synth.ensure_model(packed=True)
    toks = prompt(manifest)
    n = len(toks)
    ex = exact.ExactDecoder(Weights(d), CONTEXT, CONTEXT)
    t0 = time.time()
    bits, hidden, nxt = xp.ExactPrefill(ex).prefill(toks)
    print(f"twin prefill of {n} tokens: {time.time() - t0:.0f} s, next {nxt}", flush=True)
    out = {
        "prompt_tokens": n, "context": CONTEXT, "model_sha256": model_sha,
        "layers": [{"keys": sha(ex.keys[i][:n], np.uint16), "values": sha(ex.values[i][:n], np.uint16)}
                   for i in range(16)],
        "logits": sha(bits, np.uint16), "hidden": sha(np.asarray(hidden, np.float32).view(np.uint32), np.uint32),
        "next": int(nxt),
    }
    path = sys.argv[1] if len(sys.argv) > 1 else OUT
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print("wrote", path, flush=True)


if __name__ == "__main__":
    main()
