"""Single-token prompts whose prefill prediction is an end token: tests/golden/eos_prompts.json.

The synthetic seed-0 model has random weights, so a greedy continuation almost never meets
the end ids 1 / 16 (Main.swift:278) by itself.  Document-ordering tests need documents that
stop; a one-token prompt whose prediction is an end id stops at once (zero tokens, "stop").
This script prefills every token id as a one-token prompt on the GPU and records those whose
prediction is 1 or 16.  Tests re-check the property live before relying on it.

    python tests/golden/find_eos_prompts.py [OUT]   # on a GPU host, from the repository root
"""
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
OUT = os.path.join(ROOT, "tests", "golden", "eos_prompts.json")


def main():
    sys.path[:0] = [ROOT, os.path.join(ROOT, "plamo3-0.8b-runtime_amd")]
    import plamo_hip
    from plamo_hip import synth
    d, sha = synth.ensure_model(packed=False)
    rt = plamo_hip.Runtime(d, 64)
    found = []
    t0 = time.time()
    for t in range(plamo_hip.VOCAB):
        rt.reset()
        nxt = rt.prefill([t])
        if nxt in (1, 16):
            found.append([t, nxt])
            print("token", t, "->", nxt, flush=True)
        if t % 10000 == 0:
            print(f"{t} prompts, {time.time() - t0:.0f} s", flush=True)
    rt.close()
    out = sys.argv[1] if len(sys.argv) > 1 else OUT
    with open(out, "w") as f:
        json.dump({"synthetic_model_sha256": sha, "path": "Runtime.prefill", "eos_prompts": found}, f, indent=1)
    print("wrote", out, len(found), "prompts", flush=True)


if __name__ == "__main__":
    main()
