"""Writes tests/golden/manifest.json: the synthetic model identity and oracle vectors.

Run from the repository root:  python tests/golden/make_golden.py
The vectors come from the CPU oracle (oracle/model.py) on the seed-0 synthetic model
(plamo_hip.synth).  Tests compare the oracle against them (pinning its stability) and the
GPU path against the live oracle.
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "plamo3-0.8b-runtime_amd")]

from plamo_hip import synth  # noqa: E402
from oracle import model as om  # noqa: E402
from oracle import sampler  # noqa: E402


def prompt(config, n):
    """Uniform random non-special prompt IDs (1024..107519) from default_rng(config)."""
    return np.random.default_rng(config).integers(1024, 107520, n).tolist()


def main():
    d, sha = synth.ensure_model(packed=False)
    w = om.Weights(d)
    out = {"synthetic_model": {"seed": 0, "std": 0.02, "sha256": sha}}
    # C1: 64-token prompt, 32 greedy tokens (prefill + 31 forwards), context 96
    p1 = prompt(1, 64)
    o = om.Oracle(w, context=96)
    ids, reason = om.greedy(o, p1, 32)
    o2 = om.Oracle(w, context=96)
    o2.prefill(p1)
    lg = o2.logits_fp32.numpy()
    top = np.argsort(-lg, kind="stable")[:8]
    out["config1"] = {"prompt": p1, "greedy_ids": ids, "stop_reason": reason,
                      "prefill_top8_ids": top.tolist(), "prefill_top8_logits": lg[top].tolist(),
                      "prefill_logit_l2": float(np.linalg.norm(lg))}
    # sampling controls over generated-only history (Main.swift:237-244)
    o3 = om.Oracle(w, context=96)
    sid, sreason = om.greedy(o3, p1, 24, sampling=dict(penalty=1.1, frequency=0.2, ngram=4))
    out["config1_sampling"] = {"penalty": 1.1, "frequency": 0.2, "ngram": 4, "max_tokens": 24, "ids": sid,
                               "stop_reason": sreason}
    path = os.path.join(ROOT, "tests", "golden", "manifest.json")
    with open(path + ".part", "w") as f:
        json.dump(out, f, indent=1)
    os.replace(path + ".part", path)
    print(json.dumps({k: (v if k != "config1" else {"greedy_ids": v["greedy_ids"]}) for k, v in out.items()}))


if __name__ == "__main__":
    main()
