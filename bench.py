"""Benchmark of the PLaMo-3 0.8B token loop on one MI355X.

Headline (the JSON line's `value`): batch-1 greedy decode tokens/s of the full 16-layer model
with plain BF16 weights (BASELINE.json configs[0] shape, random-init weights, synthetic prompt),
each step one replay of the captured decode graph with the next token fed back on the device.
Extra fields: packed (.p12) decode, batch4 aggregate decode, 2048-token prefill with MFMA
utilisation, the per-projection GEMV microbenchmark and the CPU oracle baseline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "plamo3-0.8b-runtime_amd")]

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
SHAPES = {"qkv": (2304, 1536), "o": (1536, 2048), "gate_up": (12288, 1536), "down": (1536, 6144),
          "head": (107520, 1536)}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kv_read_bytes(pos):
    """K+V bytes the 16 layers read at position `pos` (14 local <= 2048 keys, 2 global)."""
    return 512 * (14 * min(pos + 1, 2048) + 2 * (pos + 1))


def gemv_microbench(torch, native, repeats=50):
    """each projection shape, plain and .p12, timed with HIP events on the stream."""
    import numpy as np
    from plamo_hip import synth  # noqa: F401  (same package, ensures path)
    lib = native.load()
    out = {}
    rng = np.random.default_rng(0)
    stream = torch.cuda.current_stream()
    for name, (m, n) in SHAPES.items():
        w = rng.standard_normal((m, n), dtype=np.float32) * np.float32(0.02)
        u = w.view(np.uint32)
        bits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        payload, entries = native.pack_tensor(bits)
        x = torch.randn(n, device="cuda").to(torch.bfloat16).float()
        wd = torch.from_numpy(bits.view(np.int16)).cuda()
        pd = torch.from_numpy(payload).cuda()
        td = torch.from_numpy(entries.view(np.int32)).cuda()
        mode = 2 if name == "head" else 0
        y = torch.empty(m, dtype=torch.float32, device="cuda")
        res = {}
        for kind, wp, tp, nbytes in (("plain", wd.data_ptr(), 0, m * n * 2),
                                     ("p12", pd.data_ptr(), td.data_ptr(), payload.nbytes + entries.nbytes)):
            for _ in range(5):
                lib.plamo_kernel_linear(wp, tp, x.data_ptr(), y.data_ptr(), n, m, 1, mode, stream.cuda_stream)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(repeats):
                lib.plamo_kernel_linear(wp, tp, x.data_ptr(), y.data_ptr(), n, m, 1, mode, stream.cuda_stream)
            e1.record(stream)
            e1.synchronize()
            us = e0.elapsed_time(e1) * 1000.0 / repeats
            res[kind] = {"us": round(us, 2), "bytes": int(nbytes), "GBps": round(nbytes / us / 1e3, 1),
                         "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 3)}
        out[name] = res
    return out


def cpu_baseline(model_dir, prompt, decode_tokens):
    """The CPU oracle (PyTorch FP32, BF16 rounding) on the host cores: bounded sample."""
    import torch
    from oracle import model as om
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    w = om.Weights(model_dir)
    o = om.Oracle(w, context=len(prompt) + decode_tokens + 1)
    t0 = time.perf_counter()
    nxt = o.prefill(prompt)
    t1 = time.perf_counter()
    for _ in range(decode_tokens):
        nxt = o.forward([nxt])
    t2 = time.perf_counter()
    return {"value": round(decode_tokens / (t2 - t1), 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"oracle/model.py FP32 CPU: {len(prompt)}-token prefill ({t1 - t0:.2f} s) then "
                      f"{decode_tokens} batch-1 decode steps of the full model"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--quick", action="store_true", help="skip the secondary measurements")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one MI355X; multi-GPU runs are not part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import numpy as np
    import torch
    import plamo_hip
    from plamo_hip import native, synth

    native.load()
    log("model: generating/packing synthetic seed-0 weights")
    model_dir, sha = synth.ensure_model(packed=True)
    prompt = np.random.default_rng(1).integers(1024, 107520, 64).tolist()
    ctx = 64 + args.warmup + args.steps + 8
    results = {}

    # --- batch-1 decode, plain and packed
    for packed in (False, True):
        rt = plamo_hip.Runtime(model_dir, ctx, packed=packed, source_sha256=sha)
        rt.prefill(prompt)
        if args.warmup:
            rt.bench_decode(max(2, args.warmup))
        start_pos = rt.position
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ms = rt.bench_decode(args.steps)
        wall = time.perf_counter() - t0
        st = rt.stats()
        mid = start_pos + args.steps // 2
        step_bytes = st["linear_bytes"] + kv_read_bytes(mid) + 16 * 512
        results["packed" if packed else "plain"] = {
            "ms_per_step": ms, "tok_s": 1000.0 / ms, "wall_s": wall, "linear_bytes": st["linear_bytes"],
            "step_bytes": step_bytes, "step_GBps": step_bytes / ms / 1e6,
            "hbm_frac": step_bytes / ms / 1e6 / HBM_PEAK_GBS}
        log(f"decode {'p12' if packed else 'bf16'}: {ms:.3f} ms/step {1000 / ms:.1f} tok/s")
        rt.close()

    # --- batch4 aggregate (4 lanes, one weight pass per step)
    if not args.quick:
        rt = plamo_hip.Runtime(model_dir, 64 + 128 + 8)
        b = plamo_hip.Batch(rt)
        prompts = [np.random.default_rng(10 + i).integers(1024, 107520, n).tolist() for i, n in
                   enumerate((64, 48, 32, 16))]
        toks = b.prefill(prompts)
        for _ in range(4):
            toks = b.step(toks)
        torch.cuda.synchronize()
        n = 100
        t0 = time.perf_counter()
        for _ in range(n):
            toks = b.step(toks)
        dt = time.perf_counter() - t0
        results["batch4"] = {"steps": n, "ms_per_step": dt * 1000 / n, "aggregate_tok_s": 4 * n / dt}
        # the same host-driven loop at batch 1 for a like-for-like ratio
        rt.reset()
        t = rt.prefill(prompts[0])
        for _ in range(4):
            t = rt.forward([t])
        t0 = time.perf_counter()
        for _ in range(n):
            t = rt.forward([t])
        dt1 = time.perf_counter() - t0
        results["batch4"]["host_loop_bs1_tok_s"] = n / dt1
        results["batch4"]["ratio_vs_bs1_host_loop"] = results["batch4"]["aggregate_tok_s"] / (n / dt1)
        log(f"batch4: {results['batch4']}")
        b.close()
        rt.close()

    # --- prefill of 2048 tokens
    if not args.quick:
        rt = plamo_hip.Runtime(model_dir, 2048 + 64)
        p2 = np.random.default_rng(3).integers(1024, 107520, 2048).tolist()
        rt.prefill(p2)
        rt.reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        rt.prefill(p2)
        dt = time.perf_counter() - t0
        gemm_flop = 2 * 34996224 * 16 * 2048
        attn_flop = 4 * 16 * 128 * sum(t + 1 for t in range(2048)) * 16
        results["prefill2048"] = {"s": dt, "tok_s": 2048 / dt, "gemm_tflop": gemm_flop / 1e12,
                                  "attn_tflop": attn_flop / 1e12,
                                  "overall_TFLOPs": (gemm_flop + attn_flop) / dt / 1e12,
                                  "mfma_frac_overall": (gemm_flop + attn_flop) / dt / 1e12 / BF16_PEAK_TFLOPS}
        log(f"prefill2048: {results['prefill2048']}")
        rt.close()

    # --- GEMV microbenchmark; the dominant decode kernel's roofline
    gemv = gemv_microbench(torch, native)
    results["gemv"] = gemv
    log(f"gemv: {json.dumps(gemv)}")
    dom = gemv["gate_up"]["plain"]

    cpu = None
    if not args.no_cpu:
        log("cpu baseline: oracle on host cores")
        cpu = cpu_baseline(model_dir, prompt, 8)

    plain = results["plain"]
    line = {
        "metric": "decode tok/s @bs1 (plain BF16, full 16-layer step, HBM roofline)",
        "value": round(plain["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(plain["ms_per_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 (fp32 accumulate)",
        "data": "synthetic: random-init N(0,0.02) BF16 weights (seed 0), uniform random 64-token prompt",
        "config": {"workload": "configs[0]/[1]: batch-1 greedy decode of the PLaMo-3 0.8B-shaped model "
                               "(hidden 1536, 16 layers, MQA 16x128, inter 6144, vocab 107520), "
                               f"64-token prompt then {args.steps} graph-replayed steps",
                   "global_batch": 1, "seq_len": ctx, "parallelism": "single GPU"},
        "step_hbm_frac": round(plain["hbm_frac"], 4),
        "roofline": {"bound": "hbm", "achieved": dom["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "gemv gate_up 12288x1536 BF16 (37,748,736 B per launch)"},
        "cpu_baseline": cpu,
        "details": results,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
