"""Benchmark of the PLaMo-3 0.8B token loop on one MI355X.

Headline (the JSON line's `value`): batch-1 greedy decode tokens/s of the full 16-layer model
with plain BF16 weights (BASELINE.json metric "decode tok/s @bs1 ... % HBM roofline"; the
configs[0] model shape, random-init weights, synthetic 64-token prompt), each step one replay
of the captured decode graph with the next token fed back on the device, timed with HIP
events on the runtime's stream.  Extra fields cover the rest of the metric and the other
configs: .p12 decode; configs[1] GEMV shapes (plain and .p12, weights cycled through more
copies than the 256 MB memory-side cache holds); configs[2] 2048-token prefill with MFMA
utilisation; configs[3] batch4 segments (512/384/256/128-token prompts, up to 2048 tokens
each, stop on EOS) against batch-1 on the same segment; configs[4] .p12 long context
(30,720-token prefill, then sampled decode to the 32,768 cap); the CPU oracle baseline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
    python bench.py --kernels-only     # GEMV shapes + copy calibration (for rocprofv3 --pmc)
    python bench.py --prefill-only     # three 2048-token prefills (for rocprofv3 kernel traces)
    python bench.py --batch4-only      # the configs[3] batch4 measurement alone
    python bench.py --long-only N      # configs[4]: 30,720-token prefill, then N sampled tokens
    python bench.py --tokenizer-only   # host C++ tokenizer throughput (no GPU work)
    python bench.py --timeline [--packed]  # in-step kernel durations of replayed decode steps
                                           # (needs lib/libplamo_hip_timeline.so: make timeline)
"""
import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "plamo3-0.8b-runtime_amd")]

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
SHAPES = {"qkv": (2304, 1536), "o": (1536, 2048), "gate_up": (12288, 1536), "down": (1536, 6144),
          "head": (107520, 1536)}
DOMINANT = "gate_up"  # largest share of the decode step's kernel time (profiles/)
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemv_gate_up_hbm_traffic.md")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kv_read_bytes(pos):
    """K+V bytes the 16 layers read at position `pos` (14 local <= 2048 keys, 2 global)."""
    return 512 * (14 * min(pos + 1, 2048) + 2 * (pos + 1))


def gemv_microbench(torch, native, repeats=48):
    """each projection shape, plain and .p12, one activation row, HIP events on
    the launch stream.  Each shape cycles through enough copies of its weights (> 512 MB) that
    every launch streams from HBM, as in the decode step."""
    import numpy as np
    lib = native.load()
    out = {}
    rng = np.random.default_rng(0)
    stream = torch.cuda.current_stream()
    for name, (m, n) in SHAPES.items():
        w = rng.standard_normal((m, n), dtype=np.float32) * np.float32(0.02)
        u = w.view(np.uint32)
        bits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        payload, entries = native.pack_tensor(bits)
        copies = max(2, -(-512 * 2 ** 20 // bits.nbytes))
        x = torch.randn(n, device="cuda").to(torch.bfloat16).float()
        wd = torch.from_numpy(bits.view(np.int16)).cuda()
        pd = torch.from_numpy(payload).cuda()
        td = torch.from_numpy(entries.view(np.int32)).cuda()
        wds = [wd] + [wd.clone() for _ in range(copies - 1)]
        pds = [(pd, td)] + [(pd.clone(), td.clone()) for _ in range(copies - 1)]
        mode = 2 if name == "head" else 0
        y = torch.empty(m, dtype=torch.float32, device="cuda")
        res = {"copies": copies}
        for kind, nbytes in (("plain", m * n * 2), ("p12", payload.nbytes + entries.nbytes)):
            def launch(i):
                if kind == "plain":
                    wp, tp = wds[i % copies].data_ptr(), 0
                else:
                    wp, tp = pds[i % copies][0].data_ptr(), pds[i % copies][1].data_ptr()
                rc = lib.plamo_kernel_linear(wp, tp, x.data_ptr(), y.data_ptr(), n, m, 1, mode, stream.cuda_stream)
                assert rc == 0
            for i in range(2 * copies):
                launch(i)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for i in range(repeats):
                launch(i)
            e1.record(stream)
            e1.synchronize()
            us = e0.elapsed_time(e1) * 1000.0 / repeats
            res[kind] = {"us": round(us, 2), "bytes": int(nbytes), "GBps": round(nbytes / us / 1e3, 1),
                         "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 3)}
        out[name] = res
        del wds, pds
    return out


def copy_calibration(torch):
    """A plain device copy of known size, for scaling the profiler's FETCH/WRITE_SIZE counters."""
    a = torch.empty(64 * 2 ** 20, dtype=torch.int32, device="cuda").fill_(1)
    b = torch.empty_like(a)
    for _ in range(4):
        b.copy_(a)
    torch.cuda.synchronize()
    return {"bytes": a.numel() * 4, "launches": 4}


def traffic_from_profile():
    """HBM bytes per launch of the dominant GEMV, from the committed rocprofv3 --pmc summary."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", f.read())
        return int(m.group(1)) if m else None
    except OSError:
        return None


def cpu_model_name():
    """The host CPU's model name (what `lscpu` prints as "Model name")."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(model_dir, prompt, decode_tokens, runs=3):
    """The CPU oracle (PyTorch FP32, BF16 rounding) on the host cores, bounded: configs[0]'s
    64-token prefill and `decode_tokens` batch-1 decode steps, `runs` warm runs each (median),
    and configs[1]'s GEMV shapes as FP32 matrix-vector products of the BF16-valued weights."""
    import statistics
    import numpy as np
    import torch
    from oracle import model as om
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    w = om.Weights(model_dir)
    o = om.Oracle(w, context=len(prompt) + decode_tokens + 1)
    o.prefill(prompt)  # warm-up
    pre, dec = [], []
    for _ in range(runs):
        o.reset()
        t0 = time.perf_counter()
        nxt = o.prefill(prompt)
        t1 = time.perf_counter()
        for _ in range(decode_tokens):
            nxt = o.forward([nxt])
        t2 = time.perf_counter()
        pre.append(t1 - t0)
        dec.append((t2 - t1) / decode_tokens)
    gemv = {}
    rng = np.random.default_rng(0)
    for name, (m, n) in SHAPES.items():
        wt = torch.from_numpy((rng.standard_normal((m, n), dtype=np.float32) * np.float32(0.02)))
        wt = wt.to(torch.bfloat16).float()
        x = torch.randn(n).to(torch.bfloat16).float()
        torch.mv(wt, x)
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            torch.mv(wt, x)
            ts.append(time.perf_counter() - t0)
        gemv[name] = round(statistics.median(ts) * 1e6, 1)
        del wt
    step = statistics.median(dec)
    return {"value": round(1.0 / step, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model_name(),
            "prefill_s": round(statistics.median(pre), 3), "decode_step_s": round(step, 4),
            "gemv_us": gemv, "runs": runs,
            "sample": f"oracle/model.py FP32 CPU, median of {runs} warm runs: {len(prompt)}-token prefill "
                      f"then {decode_tokens} batch-1 decode steps of the full model (configs[0]); "
                      "configs[1] GEMV shapes as FP32 torch.mv of BF16-valued weights"}


def bench_batch4(plamo_hip, np, model_dir):
    """four segments, prompts of 512/384/256/128 random tokens, each decoding up to
    2048 tokens (stop on EOS ids 1 / 16), one weight pass per step for all active lanes."""
    lengths, limit = (512, 384, 256, 128), 2048
    prompts = [np.random.default_rng(20 + i).integers(1024, 107520, n).tolist() for i, n in enumerate(lengths)]
    rt = plamo_hip.Runtime(model_dir, 512 + limit + 8)
    b = plamo_hip.Batch(rt)
    b.generate([p[:16] for p in prompts], [8] * 4)  # warm-up (graph capture)
    b.reset()
    t0 = time.perf_counter()
    outs = b.generate(prompts, [limit] * 4)
    dt = time.perf_counter() - t0
    produced = sum(len(ids) for ids, _ in outs)
    # batch 1 on segment 0 with the same device loop, same limit
    rt.reset()
    rt.generate(prompts[0][:16], 8)
    rt.reset()
    t0 = time.perf_counter()
    ids1, _ = rt.generate(prompts[0], limit)
    dt1 = time.perf_counter() - t0
    b.close()
    rt.close()
    res = {"segments": [len(ids) for ids, _ in outs], "reasons": [r for _, r in outs], "tokens": produced,
           "s": round(dt, 4), "aggregate_tok_s": round(produced / dt, 1),
           "bs1_same_segment_tok_s": round(len(ids1) / dt1, 1), "bs1_tokens": len(ids1)}
    res["ratio_vs_bs1"] = round(res["aggregate_tok_s"] / res["bs1_same_segment_tok_s"], 3)
    return res


def bench_long(plamo_hip, np, model_dir, sha, tokens=32768 - 30720):
    """.p12 weights, 30,720-token prefill, then sampled decode (repetition 1.1,
    frequency 0.2, no-repeat-ngram 4, on the GPU) to the 32,768-token cap (or `tokens`
    generated tokens).  Both phases are timed inside the one generate call (the runtime's
    prefill / decode wall seconds, as Main.swift:245-287 times them)."""
    rt = plamo_hip.Runtime(model_dir, 32768, packed=True, source_sha256=sha)
    prompt = np.random.default_rng(5).integers(1024, 107520, 30720).tolist()
    rt.prefill(prompt[:2048])  # warm-up
    rt.reset()
    rt.set_sampling(1.1, 0.2, 0.0, 4)
    ids, reason = rt.generate(prompt, tokens)
    st = rt.stats()
    rt.set_sampling()
    rt.close()
    t_pre, t_dec = st["last_prefill_seconds"], max(st["last_decode_seconds"], 1e-9)
    return {"prefill_tokens": 30720, "prefill_s": round(t_pre, 4), "prefill_tok_s": round(30720 / t_pre, 1),
            "decode_tokens": len(ids), "stop": reason, "decode_s": round(t_dec, 4),
            "decode_tok_s": round(len(ids) / t_dec, 1), "gpu_s": round(st["gpu_seconds"], 4)}


def bench_adapters(plamo_hip, np, model_dir, sha):
    """The trained-adapter options on random-init adapters (their acceptance and selection
    quality mean nothing here; the costs do): batch-1 decode ms/step at position 8,192 with
    QSA at budgets 2048 and 512 against dense attention (Runtime.swift:378-418), and the MTP
    draft and a two-row sequential verification against two scalar decode steps
    (Runtime.swift:322-538), each timed with HIP events around the call."""
    prompt = np.random.default_rng(6).integers(1024, 107520, 8192).tolist()
    out = {"position": 8192}
    for name, budget in (("dense", None), ("qsa2048", 2048), ("qsa512", 512)):
        rt = plamo_hip.Runtime(model_dir, 8192 + 96, source_sha256=sha, qsa_budget=budget)
        rt.prefill(prompt)
        rt.bench_decode(8)
        out[name + "_ms_per_step"] = round(rt.bench_decode(64), 4)
        rt.close()
    rt = plamo_hip.Runtime(model_dir, 2048 + 64, source_sha256=sha, mtp=True)
    nxt = rt.prefill(prompt[:2048])
    draft, verify, scalar = [], [], []
    gpu = lambda: rt.stats()["gpu_seconds"]
    for _ in range(10):
        g0 = gpu()
        d = rt.draft(nxt)[0]
        g1 = gpu()
        rt.forward([nxt, d], all=True, sequential=True)
        g2 = gpu()
        rt.rewind(rt.position - 1, 0)  # keep the first row
        nxt = rt.predictions()[0]
        g3 = gpu()
        nxt = rt.forward([rt.forward([nxt])])
        g4 = gpu()
        draft.append(g1 - g0)
        verify.append(g2 - g1)
        scalar.append(g4 - g3)
    rt.close()
    out.update({"mtp_draft_ms": round(1e3 * float(np.median(draft)), 4),
                "mtp_verify_two_rows_ms": round(1e3 * float(np.median(verify)), 4),
                "two_scalar_steps_ms": round(1e3 * float(np.median(scalar)), 4)})
    return out


def bench_tokenizer(plamo_hip, synth):
    """Host-side tokenizer (Tokenizer.swift): load, encode and decode throughput of the native
    library on ~1 MB of seeded text over the synthetic vocabulary's alphabet (no GPU work)."""
    import random
    path, alphabet = synth.ensure_tokenizer()
    t0 = time.perf_counter()
    tok = plamo_hip.Tokenizer(path)
    load = time.perf_counter() - t0
    rng = random.Random(7)
    words = ["".join(rng.choice(alphabet) for _ in range(rng.randint(1, 9))) for _ in range(4096)]
    text = " ".join(rng.choice(words) for _ in range(160000))[:1 << 20]
    nbytes = len(text.encode())
    enc, dec = [], []
    for _ in range(3):
        t0 = time.perf_counter()
        ids = tok.encode(text)
        enc.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        out = tok.decode_bytes(ids)
        dec.append(time.perf_counter() - t0)
    assert out == text.encode(), "tokenizer round trip"
    tok.close()
    return {"load_s": round(load, 3), "text_bytes": nbytes, "tokens": len(ids),
            "encode_MBps": round(nbytes / min(enc) / 1e6, 2), "encode_tok_s": round(len(ids) / min(enc)),
            "decode_MBps": round(nbytes / min(dec) / 1e6, 2), "cores": 1}


def step_timeline(plamo_hip, np, model_dir, sha, packed, steps=24):
    """In-step kernel durations of graph-replayed decode steps (positions 80-128 after a
    64-token prompt), from the device timestamps of the timeline library: each kernel's span
    (first workgroup start to last workgroup end), the gaps between consecutive kernels, and
    the step span, averaged over `steps` single-step replays."""
    rt = plamo_hip.Runtime(model_dir, 64 + 16 + 2 * steps + 8, packed=packed, source_sha256=sha)
    rt.prefill(np.random.default_rng(1).integers(1024, 107520, 64).tolist())
    rt.bench_decode(16)
    plamo_hip.timeline(clear=True)
    spans, gaps, steps_us, event_ms = {}, [], [], []
    for _ in range(steps):
        # two replays: the first (untimed, with the loop's step_begin) sets up, the second is
        # timed with HIP events and rewrites every slot but step_begin's, which is skipped
        event_ms.append(rt.bench_decode(2))
        t = plamo_hip.timeline(clear=True).astype(np.int64)
        ran = []
        for tag in range(plamo_hip.TIMELINE_TAGS):
            if tag == 251:
                continue
            blk = t[tag][t[tag][:, 0] > 0]
            if len(blk):
                ran.append((int(blk[:, 0].min()), int(blk[:, 1].max()), tag))
        ran.sort()
        for (s0, e0, tag) in ran:
            name = plamo_hip.timeline_name(tag)
            kind = name.split(".")[-1]
            spans.setdefault(kind, []).append((e0 - s0) / 100.0)  # 100 MHz ticks -> us
        gaps += [(ran[i + 1][0] - ran[i][1]) / 100.0 for i in range(len(ran) - 1)]
        steps_us.append((ran[-1][1] - ran[0][0]) / 100.0)
    rt.close()
    res = {k: {"mean_us": round(float(np.mean(v)), 3), "launches_per_step": len(v) // steps}
           for k, v in sorted(spans.items())}
    return {"packed": packed, "steps": steps, "kernels": res,
            "kernels_per_step": sum(r["launches_per_step"] for r in res.values()),
            "kernel_us_per_step": round(sum(float(np.sum(v)) for v in spans.values()) / steps, 2),
            "gap_mean_us": round(float(np.mean(gaps)), 3), "gap_min_us": round(float(np.min(gaps)), 3),
            "step_span_us": round(float(np.mean(steps_us)), 2),
            "event_ms_per_step": round(float(np.mean(event_ms)), 4)}


def timeline_child(packed):
    """step_timeline in a child process that loads lib/libplamo_hip_timeline.so (this process
    holds the normal library); None when that library is not built."""
    import subprocess
    from plamo_hip import native
    if not os.path.exists(native.TIMELINE_LIB_PATH):
        return None
    cmd = [sys.executable, os.path.abspath(__file__), "--timeline"] + (["--packed"] if packed else [])
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    if out.returncode != 0:
        log(out.stderr[-2000:])
        return None
    return json.loads(out.stdout.strip().splitlines()[-1])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--quick", action="store_true", help="skip the secondary measurements")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernels-only", action="store_true", help="GEMV shapes and a copy calibration only")
    ap.add_argument("--prefill-only", action="store_true", help="three 2048-token prefills only")
    ap.add_argument("--batch4-only", action="store_true", help="the configs[3] batch4 measurement only")
    ap.add_argument("--long-only", type=int, default=0, metavar="TOKENS",
                    help="the configs[4] workload only, generating TOKENS tokens after the 30,720-token prefill")
    ap.add_argument("--tokenizer-only", action="store_true",
                    help="host tokenizer throughput (no GPU work; not part of the GPU line)")
    ap.add_argument("--timeline", action="store_true",
                    help="in-step kernel durations from the timeline library (make timeline)")
    ap.add_argument("--packed", action="store_true", help="with --timeline: .p12 weights")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one MI355X; multi-GPU runs are not part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import numpy as np
    import torch
    import plamo_hip
    from plamo_hip import native, synth

    if args.timeline:
        native.LIB_PATH = native.TIMELINE_LIB_PATH
    native.load()
    if args.timeline:
        model_dir, sha = synth.ensure_model(packed=True)
        print(json.dumps(step_timeline(plamo_hip, np, model_dir, sha, args.packed)), flush=True)
        return
    if args.kernels_only:
        gemv = gemv_microbench(torch, native)
        cal = copy_calibration(torch)
        print(json.dumps({"gemv": gemv, "copy_calibration": cal}), flush=True)
        return
    log("model: generating/packing synthetic seed-0 weights")
    model_dir, sha = synth.ensure_model(packed=True)
    if args.batch4_only:
        print(json.dumps({"batch4": bench_batch4(plamo_hip, np, model_dir)}), flush=True)
        return
    if args.long_only:
        print(json.dumps({"long_context": bench_long(plamo_hip, np, model_dir, sha, args.long_only)}), flush=True)
        return
    if args.tokenizer_only:
        print(json.dumps({"tokenizer": bench_tokenizer(plamo_hip, synth)}), flush=True)
        return
    if args.prefill_only:
        rt = plamo_hip.Runtime(model_dir, 2048 + 64)
        p2 = np.random.default_rng(3).integers(1024, 107520, 2048).tolist()
        for _ in range(3):
            rt.reset()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            rt.prefill(p2)
            log(f"prefill 2048: {(time.perf_counter() - t0) * 1e3:.2f} ms")
        rt.close()
        return
    prompt = np.random.default_rng(1).integers(1024, 107520, 64).tolist()
    ctx = 64 + args.warmup + args.steps + 8
    results = {}

    # --- batch-1 decode, plain and packed (the headline)
    for packed in (False, True):
        rt = plamo_hip.Runtime(model_dir, ctx, packed=packed, source_sha256=sha)
        rt.prefill(prompt)
        if args.warmup:
            rt.bench_decode(max(2, args.warmup))
        start_pos = rt.position
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ms = rt.bench_decode(args.steps)
        torch.cuda.synchronize()
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

    if not args.quick:
        results["batch4"] = bench_batch4(plamo_hip, np, model_dir)
        log(f"batch4: {results['batch4']}")
        results["long_context"] = bench_long(plamo_hip, np, model_dir, sha)
        log(f"long_context: {results['long_context']}")
        results["adapters"] = bench_adapters(plamo_hip, np, model_dir, sha)
        log(f"adapters: {results['adapters']}")
        # --- prefill of 2048 tokens
        rt = plamo_hip.Runtime(model_dir, 2048 + 64)
        p2 = np.random.default_rng(3).integers(1024, 107520, 2048).tolist()
        rt.prefill(p2)
        # median of five prefills: GPU time of the runtime's stream (its gpu_seconds, as the
        # reference's Runtime.gpuSeconds) and the host's wall clock around each call
        gpu_s, wall_s = [], []
        for _ in range(5):
            rt.reset()
            torch.cuda.synchronize()
            g0 = rt.stats()["gpu_seconds"]
            t0 = time.perf_counter()
            rt.prefill(p2)
            wall_s.append(time.perf_counter() - t0)
            gpu_s.append(rt.stats()["gpu_seconds"] - g0)
        dt = float(np.median(gpu_s))
        gemm_flop = 2 * 34996224 * 16 * 2048
        attn_flop = 4 * 16 * 128 * sum(min(t + 1, 2048) for t in range(2048)) * 16
        results["prefill2048"] = {"s": dt, "wall_s": float(np.median(wall_s)), "runs": 5, "tok_s": 2048 / dt,
                                  "gemm_tflop": gemm_flop / 1e12,
                                  "attn_tflop": attn_flop / 1e12,
                                  "overall_TFLOPs": (gemm_flop + attn_flop) / dt / 1e12,
                                  "mfma_frac_overall": (gemm_flop + attn_flop) / dt / 1e12 / BF16_PEAK_TFLOPS}
        log(f"prefill2048: {results['prefill2048']}")
        rt.close()

    # --- GEMV shapes; the dominant decode kernel's roofline
    gemv = gemv_microbench(torch, native)
    results["gemv"] = gemv
    log(f"gemv: {json.dumps(gemv)}")
    dom = gemv[DOMINANT]["plain"]

    timeline = {"plain": timeline_child(False), "p12": timeline_child(True)}
    results["timeline"] = timeline
    log(f"timeline: {json.dumps(timeline)}")
    in_step = None
    if timeline["plain"] and DOMINANT in timeline["plain"]["kernels"]:
        us = timeline["plain"]["kernels"][DOMINANT]["mean_us"]
        in_step = {"us": us, "GBps": round(37748736 / us / 1e3, 1), "frac": round(37748736 / us / 1e3 / HBM_PEAK_GBS, 4),
                   "source": "device timestamps of graph-replayed steps (lib/libplamo_hip_timeline.so, "
                             "bench.py --timeline)"}

    cpu = None
    if not args.no_cpu:
        log("cpu baseline: oracle on host cores")
        cpu = cpu_baseline(model_dir, prompt, 6)

    plain = results["plain"]
    line = {
        "metric": "decode tok/s @bs1 (plain BF16, full 16-layer step, HBM roofline)",
        "value": round(plain["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(plain["ms_per_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 (fp32 accumulate)",
        "data": "synthetic: random-init N(0,0.02) BF16 weights (seed 0), uniform random 64-token prompt",
        "config": {"workload": "configs[0] model shape: batch-1 greedy decode of the PLaMo-3 0.8B-shaped "
                               "model (hidden 1536, 16 layers, MQA 16x128, inter 6144, vocab 107520), "
                               f"64-token prompt then {args.steps} graph-replayed steps",
                   "global_batch": 1, "seq_len": ctx, "parallelism": "single GPU"},
        "step_hbm_frac": round(plain["hbm_frac"], 4),
        "roofline": {"bound": "hbm", "achieved": dom["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4), "traffic": traffic_from_profile(),
                     "kernel": f"gemv {DOMINANT} 12288x1536 BF16, one row, weights streamed from HBM "
                               "(37,748,736 B per launch)",
                     "scope": "isolated launch (configs[1] shape, plain activation prologue), HIP events",
                     "in_step": in_step},
        "cpu_baseline": cpu,
        "details": results,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
