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


def trajectory_gaps(w, prompt_ids, ids, sampling, dots="fp32"):
    """The oracle's top-2 gap (FP32 logits, after the sampling adjustments when given), its
    BF16 ulp and its eight best (id, logit) at each step of its own trajectory `ids`
    (Main.swift:235-288)."""
    o = om.Oracle(w, context=96, dots=dots)
    o.prefill(prompt_ids)
    gaps, ulps, tops, hist = [], [], [], []
    for i, t in enumerate(ids):
        lg = o.logits_fp32.numpy().astype(np.float32).copy()
        if sampling:
            sampler.select(lg, hist, sampling["penalty"], sampling["ngram"], sampling["frequency"])
        top = np.argsort(-lg, kind="stable")[:8]
        gaps.append(float(lg[top[0]] - lg[top[1]]))
        ulps.append(bf16_ulp(lg[top[0]]))
        tops.append([[int(k), float(lg[k])] for k in top])
        hist.append(t)
        if i + 1 < len(ids):
            o.forward([t])
    return {"top2_gaps": gaps, "top_ulps": ulps, "top8": tops}


def pair_gap_noise(w, prompt_ids, ids, sampling=None):
    """Largest change of a top-8 logit gap (best minus k-th best) between the FP32-dot and
    the exact-dot oracle, both teacher-forced along `ids`: how far two valid summation
    orders move the margin a choice is made by."""
    a, b = om.Oracle(w, context=96), om.Oracle(w, context=96, dots="exact")
    a.prefill(prompt_ids)
    b.prefill(prompt_ids)
    worst, hist = 0.0, []
    for i, t in enumerate(ids):
        la = a.logits_fp32.numpy().astype(np.float32).copy()
        lb = b.logits_fp32.numpy().astype(np.float32).copy()
        if sampling:
            for lg in (la, lb):
                sampler.select(lg, hist, sampling["penalty"], sampling["ngram"], sampling["frequency"])
        top = np.argsort(-lb, kind="stable")[:8]
        d = (la[top[0]] - la[top[1:]]) - (lb[top[0]] - lb[top[1:]])
        worst = max(worst, float(np.abs(d).max()))
        hist.append(t)
        if i + 1 < len(ids):
            a.forward([t])
            b.forward([t])
    return worst


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
    # the same trajectories with correctly rounded dots: the reference for the GPU's choices
    # (deterministic across machines; torch's FP32 sums change with the host's thread count)
    oe = om.Oracle(w, context=96, dots="exact")
    eids, ereason = om.greedy(oe, p1, 32)
    out["config1"]["exact"] = {"greedy_ids": eids, "stop_reason": ereason}
    out["config1"]["exact"].update(trajectory_gaps(w, p1, eids, None, "exact"))
    # sampling controls over generated-only history (Main.swift:237-244)
    o3 = om.Oracle(w, context=96)
    ctl = dict(penalty=1.1, frequency=0.2, ngram=4)
    sid, sreason = om.greedy(o3, p1, 24, sampling=ctl)
    out["config1_sampling"] = {"penalty": 1.1, "frequency": 0.2, "ngram": 4, "max_tokens": 24, "ids": sid,
                               "stop_reason": sreason}
    out["config1_sampling"].update(trajectory_gaps(w, p1, sid, ctl))
    oe = om.Oracle(w, context=96, dots="exact")
    esid, esreason = om.greedy(oe, p1, 24, sampling=ctl)
    out["config1_sampling"]["exact"] = {"ids": esid, "stop_reason": esreason}
    out["config1_sampling"]["exact"].update(trajectory_gaps(w, p1, esid, ctl, "exact"))
    # C3: one 2048-token prompt prefilled at once (Runtime.prefill semantics, oracle `fill`)
    p3 = prompt(3, 2048)
    o4 = om.Oracle(w, context=2048)
    n3 = o4.fill(p3)
    l3 = o4.logits_fp32.numpy()
    top3 = np.argsort(-l3, kind="stable")[:8]
    out["config3"] = {"prompt_seed": 3, "length": 2048, "next": n3, "top8_ids": top3.tolist(),
                      "top8_logits": l3[top3].tolist()}
    o5 = om.Oracle(w, context=2048, dots="exact")
    e3 = o5.fill(p3)
    le3 = o5.logits_fp32.numpy()
    etop3 = np.argsort(-le3, kind="stable")[:8]
    out["config3"]["exact"] = {"next": e3, "top8_ids": etop3.tolist(), "top8_logits": le3[etop3].tolist()}
    # summation-order noise floor: FP32 dots vs correctly rounded dots, same algorithm
    out["noise_floor"] = {"config1": floor(w, p1, 96, "prefill"), "config3": floor(w, p3, 2048, "fill"),
                          "pair_gap": pair_gap_noise(w, p1, eids)}
    path = os.path.join(ROOT, "tests", "golden", "manifest.json")
    with open(path + ".part", "w") as f:
        json.dump(out, f, indent=1)
    os.replace(path + ".part", path)
    print(json.dumps({k: v for k, v in out.items() if k in ("noise_floor", "config3")}))


if __name__ == "__main__":
    main()
