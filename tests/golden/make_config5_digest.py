"""Digests of the order-exact prefill twin on configs[4]: tests/golden/config5_prefill_digest.json.

The 30,720-token configs[4] prompt (numpy default_rng(5), ids 1024 .. 107519, as the
long-context GPU tests draw it) is prefilled by oracle/exact_prefill.py on the synthetic
seed-0 model at context 32,768 in 15 chunks of 2048 (the runtime's chunking, local rings of
4096 slots), all 16 layers, then the last token's head.  The twin takes hours of CPU, so
this script records SHA-256 digests of what it produces and the GPU test compares the device
prefill's bytes with them:

  layers[i].keys / values   the cached rows of layer i (BF16 bits, uint16 little-endian):
                            every slot of a local layer's ring, rows 0 .. n-1 of a global
                            layer;
  logits                    the last token's logits as the runtime returns them (BF16 bits);
  hidden                    the last token's final hidden row (FP32 bits);
  next                      the greedy next token.

    python tests/golden/make_config5_digest.py [OUT]   # from the repository root, CPU only
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
OUT = os.path.join(ROOT, "tests", "golden", "config5_prefill_digest.json")
CONTEXT = 32768
LOCAL = 4096


def sha(a, dtype):
    return hashlib.sha256(np.ascontiguousarray(a, dtype=dtype).tobytes()).hexdigest()


def prompt():
    return np.random.default_rng(5).integers(1024, 107520, 30720).tolist()


def main():
    sys.path[:0] = [ROOT, os.path.join(ROOT, "plamo3-0.8b-runtime_amd")]
    from oracle import exact, exact_prefill as xp
    from oracle.model import Weights
    from plamo_hip import synth
    d, model_sha = synth.ensure_model(packed=True)
    toks = prompt()
    n = len(toks)
    ex = exact.ExactDecoder(Weights(d), CONTEXT, LOCAL)
    t0 = time.time()
    bits, hidden, nxt = xp.ExactPrefill(ex).prefill(toks)
    print(f"twin prefill of {n} tokens: {time.time() - t0:.0f} s, next {nxt}", flush=True)
    out = {
        "prompt_tokens": n, "context": CONTEXT, "model_sha256": model_sha,
        "local_capacity": LOCAL,
        "layers": [{"keys": sha(ex.keys[i][:min(n, ex.cap[i])], np.uint16),
                    "values": sha(ex.values[i][:min(n, ex.cap[i])], np.uint16)} for i in range(16)],
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
