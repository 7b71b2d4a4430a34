"""Writes tests/golden/manifest.json: the synthetic model identity and oracle vectors.

Run from the repository root:  python tests/golden/make_golden.py
The vectors come from the CPU oracle (oracle/model.py) on the seed-0 synthetic model
(plamo_hip.synth).  Tests compare the oracle against them (pinning its stability) and the
GPU path against the live oracle.  Also recorded: the oracle's top-2 logit gap at every step
of its greedy and sampled trajectories (where a different summation order may legitimately
choose differently: gaps under one BF16 ulp), and the summation-order noise floor (FP32 dots
vs correctly rounded dots) after the config-1 and config-3 prompts.
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


def bf16_ulp(v):
    """Spacing of BF16 values at |v| (8 significant bits)."""
    return float(2.0 ** (np.floor(np.log2(abs(v))) - 7))


def trajectory_gaps(w, prompt_ids, ids, sampling):
    """The oracle's top-2 gap (FP32 logits, after the sampling adjustments when given) and
    its BF16 ulp at each step of its own trajectory `ids` (Main.swift:235-288)."""
    o = om.Oracle(w, context=96)
    o.prefill(prompt_ids)
    gaps, ulps, hist = [], [], []
    for i, t in enumerate(ids):
        lg = o.logits_fp32.numpy().astype(np.float32).copy()
        if sampling:
            sampler.select(lg, hist, sampling["penalty"], sampling["ngram"], sampling["frequency"])
        s = np.sort(lg)[::-1]
        gaps.append(float(s[0] - s[1]))
        ulps.append(bf16_ulp(s[0]))
        hist.append(t)
        if i + 1 < len(ids):
            o.forward([t])
    return {"top2_gaps": gaps, "top_ulps": ulps}


def floor(w, p, context, mode):
    """[max-abs, RMSE] between the FP32-dot and exact-dot oracles' logits after the prompt."""
    logits = []
    for dots in ("fp32", "exact"):
        o = om.Oracle(w, context=context, dots=dots)
        getattr(o, mode)(p)
        logits.append(o.logits_fp32.numpy().astype(np.float64))
    e = np.abs(logits[0] - logits[1])
    return [float(e.max()), float(np.sqrt(np.mean(e ** 2)))]


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
    out["config1"].update(trajectory_gaps(w, p1, ids, None))
    # sampling controls over generated-only history (Main.swift:237-244)
    o3 = om.Oracle(w, context=96)
    ctl = dict(penalty=1.1, frequency=0.2, ngram=4)
    sid, sreason = om.greedy(o3, p1, 24, sampling=ctl)
    out["config1_sampling"] = {"penalty": 1.1, "frequency": 0.2, "ngram": 4, "max_tokens": 24, "ids": sid,
                               "stop_reason": sreason}
    out["config1_sampling"].update(trajectory_gaps(w, p1, sid, ctl))
    # C3: one 2048-token prompt prefilled at once (Runtime.prefill semantics, oracle `fill`)
    p3 = prompt(3, 2048)
    o4 = om.Oracle(w, context=2048)
    n3 = o4.fill(p3)
    l3 = o4.logits_fp32.numpy()
    top3 = np.argsort(-l3, kind="stable")[:8]
    out["config3"] = {"prompt_seed": 3, "length": 2048, "next": n3, "top8_ids": top3.tolist(),
                      "top8_logits": l3[top3].tolist()}
    # summation-order noise floor: FP32 dots vs correctly rounded dots, same algorithm
    out["noise_floor"] = {"config1": floor(w, p1, 96, "prefill"), "config3": floor(w, p3, 2048, "fill")}
    path = os.path.join(ROOT, "tests", "golden", "manifest.json")
    with open(path + ".part", "w") as f:
        json.dump(out, f, indent=1)
    os.replace(path + ".part", path)
    print(json.dumps({k: v for k, v in out.items() if k in ("noise_floor", "config3")}))


if __name__ == "__main__":
    main()
