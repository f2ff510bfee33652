"""Decode throughput benchmark (one MI355X).

Headline workload: Llama-3.2-1B-shaped model with Q8_0 linear weights (FP16
embeddings, untied Q8_0 classifier), batch-1 greedy decode over positions
0-2047.  The timed steps are cut into segments of at least 32 tokens (one
persistent launch each) spread over the range; before each segment the fp16
KV cache holds N(0,1) history up to the segment's start.  `--steps K` times
exactly K tokens.  The same JSON line carries the Llama-3.1-8B-shaped Q8_0
workload (128 greedy steps at each of the 8k / 16k / 32k KV fills) with its
own roofline, the standalone attention kernel's rate at each fill, and the CPU
baseline.  Weights are random-init from a seed (no checkpoints).  One JSON
line on stdout; details on stderr.

    python bench.py [--steps 256] [--warmup 8] [--config llama1b_q8] [--schedule persistent|graph]
                    [--starts P1,P2,...] [--steps-8b 128] [--no-8b] [--no-cpu-baseline]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gpullama3.java_amd"))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

METRIC = "decode tok/s + achieved HBM GB/s (% of 8 TB/s), 1B & 8B Q8_0, batch 1"
HBM_PEAK_GBS = 8000.0
MIN_PER_LAUNCH = 32          # tokens per persistent launch the segments keep when --steps allows
FILLS_8B = (8192, 16384, 32768)
SPAN_1B = 2048               # the 1B workloads' positions 0 .. 2047


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def weight_bytes(shape, specs):
    """Linear-weight bytes streamed per token (classifier included) + one embedding row."""
    from gpullama3_hip.model import type_nbytes
    total = 0
    for sp in specs:
        if sp.name.endswith("norm.weight") or sp.name == "token_embd.weight":
            continue
        total += sp.nbytes
    if shape.tied:
        total += type_nbytes(shape.embd_type, shape.vocab_size * shape.dim)
    total += type_nbytes(shape.embd_type, shape.dim)
    return total


def kv_bytes(shape, pos, elem_bytes=2):
    """K and V of positions 0..pos, all layers (fp16 on the device; the reference's CPU cache is fp32)."""
    return 2 * shape.n_layers * shape.kv_dim * elem_bytes * (pos + 1)


def split_steps(steps, nseg):
    """nseg segment lengths summing to exactly `steps` (the first ones one longer)."""
    base, rem = divmod(steps, nseg)
    return [base + (1 if i < rem else 0) for i in range(nseg)]


def segments(cfg_key, steps, ctx, starts=None):
    """(start, n) segments of exactly `steps` tokens in total.

    Given starts: the steps are split over them.  Llama-3.1-8B: split over its
    three fills.  Otherwise min(8, steps // 32) segments (at least one) with
    starts spread over the workload's span so the mean position is the span's
    middle; every segment holds >= 32 tokens whenever steps >= 32."""
    if steps <= 0:
        raise ValueError("--steps must be positive")
    if starts:
        return list(zip(starts, split_steps(steps, len(starts))))
    if cfg_key == "llama8b_q8":
        return list(zip(FILLS_8B, split_steps(steps, len(FILLS_8B))))
    span = SPAN_1B if cfg_key.startswith("llama1b") else min(ctx, 4096)
    nseg = max(1, min(8, steps // MIN_PER_LAUNCH))
    lens = split_steps(steps, nseg)
    if steps >= span:
        raise ValueError(f"--steps {steps} does not fit the workload span of {span} positions")
    if nseg == 1:
        return [((span - steps) // 2, steps)]
    last = span - lens[-1]
    return [(int(round(last * i / (nseg - 1))), n) for i, n in enumerate(lens)]


def cpu_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model, os.cpu_count() or 1


def cpu_threads():
    """All the cores this process may use: the CPU share the job was given
    (OMP_NUM_THREADS when set, e.g. 16 on a one-GPU box), else every core."""
    n = os.cpu_count() or 1
    try:
        n = min(n, len(os.sched_getaffinity(0)))
    except AttributeError:
        pass
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return n


def cpu_decode_rate(shape, tensors, starts, per_start, threads, budget_s=0.0):
    """The oracle (C restatement of the reference CPU forward, fp32 KV cache as the
    reference's, OpenMP over rows and heads) decoding `per_start` greedy steps
    from each start position; with budget_s, more consecutive steps from each start
    (as many as the context allows) until about budget_s seconds of decode have run.
    Returns (tok/s, tokens, seconds, algorithmic bytes)."""
    import oracle.oracle as orc
    from gpullama3_hip.model import tensor_specs
    m = orc.OracleModel(shape, tensors, n_threads=threads)
    wb = weight_bytes(shape, tensor_specs(shape))
    m.forward(1, 0)  # thread pool and page warm-up
    n, dt, nbytes = 0, 0.0, 0
    tok = 1
    taken = [0] * len(starts)

    def run(k, count):
        nonlocal n, dt, nbytes, tok
        for _ in range(count):
            p = starts[k] + taken[k]
            if p >= shape.context_length:
                return
            t0 = time.perf_counter()
            lg = m.forward(tok, p)
            dt += time.perf_counter() - t0
            tok = int(np.argmax(lg))
            n += 1
            taken[k] += 1
            nbytes += wb + kv_bytes(shape, p, elem_bytes=4)

    for k in range(len(starts)):
        run(k, per_start)
    if budget_s > dt and n > 0:
        extra = int(np.ceil((budget_s - dt) / (dt / n) / len(starts)))
        for k in range(len(starts)):
            run(k, extra)
    m.close()
    return n / dt, n, dt, nbytes


def cpu_baseline(shape, tensors, starts, per_start_all=32, per_start_one=4, budget_s=12.0):
    """CPU baseline on this host, at the GPU line's segment starts: all cores
    (the primary figure, a sample of about budget_s seconds) and one thread
    (secondary)."""
    model, nproc = cpu_info()
    thr = cpu_threads()
    v_all, n_all, t_all, b_all = cpu_decode_rate(shape, tensors, starts, per_start_all, thr, budget_s)
    v_one, n_one, t_one, b_one = cpu_decode_rate(shape, tensors, starts, per_start_one, 1)
    return {"value": round(v_all, 3), "unit": "tok/s", "cores": thr, "kind": "port",
            "sample": f"{n_all} greedy decode steps (consecutive positions from each GPU segment start "
                      f"{list(starts)}) of the same model: the oracle (C restatement of the reference CPU forward, "
                      f"fp32 KV cache, OpenMP over rows and heads, AVX2 8-lane dots), {t_all:.1f} s",
            "cpu_model": model, "nproc": nproc, "threads": thr,
            "achieved_gbs": round(b_all / t_all / 1e9, 2),
            "one_thread": {"value": round(v_one, 3), "unit": "tok/s", "steps": n_one, "seconds": round(t_one, 2),
                           "achieved_gbs": round(b_one / t_one / 1e9, 2)},
            "gbs_formula": "linear weights + fp32 K/V of positions 0..pos + one embedding row, per token"}


def copy_calibration(n_floats=256 << 20, reps=3, out=None):
    """A plain elementwise copy kernel of known size (reads and writes 4 * n_floats
    bytes per dispatch), run under rocprofv3 --pmc to scale FETCH_SIZE/WRITE_SIZE."""
    import torch
    a = torch.ones(n_floats, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    for _ in range(reps):
        torch.mul(a, 1.0, out=b)
    torch.cuda.synchronize()
    print(json.dumps({"copy_kernel": "torch.mul(a, 1.0, out=b) float32", "bytes_read_per_dispatch": 4 * n_floats,
                      "bytes_written_per_dispatch": 4 * n_floats, "dispatches": reps}), file=out or sys.stdout,
          flush=True)
    del a, b
    torch.cuda.empty_cache()


def profiled_traffic(cfg_key, tokens_per_launch):
    """HBM bytes per launch of the decode kernel taken from the committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration),
    rescaled to `tokens_per_launch`: (bytes, source file), or (None, None)."""
    rel = os.path.join("profiles", f"traffic_decode_step_{cfg_key}.txt")
    path = os.path.join(ROOT, rel)
    if not os.path.exists(path):
        return None, None
    vals = {}
    with open(path) as f:
        for line in f:
            if ":" in line and not line.startswith("#"):
                k, v = line.split(":", 1)
                vals[k.strip()] = v.strip()
    try:
        per_token = (float(vals["fetch_bytes_per_launch"]) + float(vals["write_bytes_per_launch"])) / \
            float(vals["tokens_per_launch"])
    except (KeyError, ValueError, ZeroDivisionError):
        return None, None
    return int(per_token * tokens_per_launch), rel


def run_decode(plan, shape, wbytes, segs, seed, first_token=1):
    """Greedy decode of every segment (KV history N(0,1) up to its start); wall
    time and HIP-event kernel time of the launches."""
    wall = kern_ms = 0.0
    launches = 0
    algo = 0
    per_seg = []
    tok = first_token
    for start, n in segs:
        plan.reset()
        if start > 0:
            plan.fill_kv_normal(seed + start, start)
        t1 = time.perf_counter()
        out = plan.generate_greedy(tok, start, n)
        t2 = time.perf_counter()
        _, km, nl = plan.timing()
        wall += t2 - t1
        kern_ms += km
        launches += nl
        seg_bytes = sum(wbytes + kv_bytes(shape, start + i) for i in range(n))
        algo += seg_bytes
        per_seg.append({"start": start, "tokens": n, "ms_per_token": round(1e3 * (t2 - t1) / n, 4),
                        "kernel_ms_per_token": round(km / n, 4),
                        "algorithmic_gbs": round(seg_bytes / (km * 1e-3) / 1e9, 1)})
        log(f"  segment start={start:6d} steps={n}: wall {1e3 * (t2 - t1) / n:.3f} ms/token, kernel {km / n:.3f} "
            f"ms/token over {nl} launch(es), {seg_bytes / (km * 1e-3) / 1e9:.0f} GB/s algorithmic")
        tok = int(out[-1])
    steps = sum(n for _, n in segs)
    return {"steps": steps, "wall_s": wall, "kernel_ms": kern_ms, "launches": launches, "algo_bytes": algo,
            "segments": per_seg}


def roofline(res, kernel):
    avg_kernel_s = res["kernel_ms"] * 1e-3 / res["launches"]
    avg_bytes = res["algo_bytes"] / res["launches"]
    achieved = avg_bytes / avg_kernel_s / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": kernel,
            "bytes_per_launch": int(avg_bytes), "avg_launch_ms": round(avg_kernel_s * 1e3, 4)}


def attention_rate(plan, shape, pos, reps=20):
    """Standalone flash-decode attention kernel (the per-phase schedule's) on layer 0
    at `pos` over the plan's cache: HIP-event average and KV GB/s."""
    ms = plan.time_attention(0, pos, reps)
    kv = kv_bytes(shape, pos) / shape.n_layers
    return {"position": pos, "avg_us": round(ms * 1e3, 2), "kv_bytes": int(kv),
            "achieved_gbs": round(kv / (ms * 1e-3) / 1e9, 1), "frac": round(kv / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def attention_only(seed, key="llama8b_q8", reps=50):
    """The standalone flash-decode attention kernel of the Llama-3.1-8B shape at
    each KV fill (fp16 N(0,1) history), without any decode step: a process that
    a kernel-trace profiler can follow from start to exit."""
    from gpullama3_hip import HipMasterPlan
    from gpullama3_hip import _lib as L
    from gpullama3_hip.model import CONFIGS, synth_model

    shape = CONFIGS[key].with_(n_layers=1, context_length=max(FILLS_8B) + 16)
    plan = HipMasterPlan.initialize_plan(shape, synth_model(shape, seed, norm_init="ones"),
                                         flags=L.FLAG_PHASE_KERNELS)
    out = []
    for pos in FILLS_8B:
        plan.fill_kv_normal(seed + pos, pos)
        out.append(attention_rate(plan, shape, pos, reps))
    plan.free_execution_plan()
    return {"workload": f"{key}: standalone attention kernel, one layer, {reps} launches at each KV fill",
            "attention_kernel": out}


def bench_config(key, steps, warmup, seed, schedule, starts=None, with_attention=False):
    from gpullama3_hip import HipMasterPlan
    from gpullama3_hip import _lib as L
    from gpullama3_hip.model import CONFIGS, synth_model, tensor_specs

    shape = CONFIGS[key]
    t0 = time.perf_counter()
    tensors = synth_model(shape, seed, norm_init="ones")
    log(f"{key}: synthetic weights {time.perf_counter() - t0:.1f} s")
    flags = L.FLAG_TIMING | (L.FLAG_PHASE_KERNELS if schedule == "graph" else 0)
    t0 = time.perf_counter()
    plan = HipMasterPlan.initialize_plan(shape, tensors, flags=flags)
    log(f"{key}: plan created and weights uploaded in {time.perf_counter() - t0:.1f} s")
    wbytes = weight_bytes(shape, tensor_specs(shape))
    segs = segments(key, steps, shape.context_length, starts)
    if any(s < 0 or s + n > shape.context_length for s, n in segs):
        raise SystemExit(f"segments {segs} do not fit the context of {shape.context_length} positions")
    if warmup > 0:
        plan.generate_greedy(1, 0, warmup)
    res = run_decode(plan, shape, wbytes, segs, seed)
    per_launch = res["steps"] / res["launches"]
    kernel = (f"decode_step_kernel (persistent, {per_launch:g} tokens per launch)" if schedule == "persistent"
              else "hipGraph of phase kernels (one replay per token)")
    rl = roofline(res, kernel)
    if schedule == "persistent":
        tr, src = profiled_traffic(key, per_launch)
        rl["traffic"] = tr
        rl["traffic_source"] = (f"copied from {src}: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of this workload, "
                                f"calibrated by a copy kernel, rescaled to {per_launch:g} tokens per launch"
                                if src else None)
    out = {"shape": shape, "tensors": tensors, "plan": plan, "segs": segs, "res": res, "roofline": rl,
           "tok_s": res["steps"] / res["wall_s"]}
    if with_attention:
        att = []
        for pos in FILLS_8B if key == "llama8b_q8" else (segs[-1][0],):
            if pos < shape.context_length:
                plan.fill_kv_normal(seed + pos, pos)
                att.append(attention_rate(plan, shape, pos))
                log(f"  attention kernel at {pos}: {att[-1]['avg_us']} us per layer, {att[-1]['achieved_gbs']} GB/s")
        out["attention"] = att
    return out


def reference_workload(plan, shape, seed):
    """The reference's own workload shape and count: a 128-token random prompt,
    then 128 greedy tokens from position 0, tokens/s = (prompt + generated) /
    wall time (InferenceEngine.java:134-138); prompt and generation on the device."""
    plan.reset()
    prompt = np.random.default_rng(seed).integers(0, shape.vocab_size, 128)
    plan.generate_from_prompt(prompt, 0, 4)  # warm the path
    plan.reset()
    t1 = time.perf_counter()
    plan.generate_from_prompt(prompt, 0, 128)
    t2 = time.perf_counter()
    return {"prompt_tokens": 128, "generated_tokens": 128, "tok_s": round(256 / (t2 - t1), 2),
            "wall_ms": round(1e3 * (t2 - t1), 3),
            "note": "(prompt + generated) / wall time from position 0, as the reference counts its tok/s"}


def reference_workload_sampled(plan, shape, seed, temperature=0.1, topp=0.95):
    """The same workload with the reference's default sampler (temperature 0.1,
    top-p 0.95: Options.java:54-55), sampled on the device (gl3_generate_sampled)
    with seeded draws in place of rng.nextFloat(1f)."""
    plan.reset()
    prompt = np.random.default_rng(seed).integers(0, shape.vocab_size, 128)
    coins = np.random.default_rng(seed + 1).random(128).astype(np.float32)
    plan.generate_sampled(prompt, 0, 4, temperature, topp, coins)  # warm the path
    plan.reset()
    t1 = time.perf_counter()
    plan.generate_sampled(prompt, 0, 128, temperature, topp, coins)
    t2 = time.perf_counter()
    return {"prompt_tokens": 128, "generated_tokens": 128, "temperature": temperature, "topp": topp,
            "tok_s": round(256 / (t2 - t1), 2), "wall_ms": round(1e3 * (t2 - t1), 3),
            "note": "on-device top-p sampling, one launch per generated token plus the sampler"}


def prefill_flops(shape, n, pos0=0):
    """Algorithmic flops of n prompt tokens at positions pos0..: the four matrix
    products of every layer (2 flops per weight per token) and causal attention
    (scores and weighted sum: 4 * head_dim flops per head per cached position)."""
    s = shape
    per_tok = 2 * (s.dim * (s.q_dim + 2 * s.kv_dim) + s.q_dim * s.dim + 2 * s.dim * s.hidden_dim + s.hidden_dim * s.dim)
    positions = sum(pos0 + i + 1 for i in range(n))
    return s.n_layers * (per_tok * n + 4 * s.head_dim * s.n_heads * positions)


def prompt_workload(seed, key="qwen3_06b_q8", n_prompt=512, n_gen=256, stepwise=True):
    """Qwen3-0.6B Q8_0 with a 512-token random prompt and 256 greedy tokens
    from position 0, tokens/s = (prompt + generated) / wall time as the
    reference counts it: the prompt through the batched prefill, and the same
    call with the prompt forwarded one decode step per token."""
    from gpullama3_hip import HipMasterPlan
    from gpullama3_hip import _lib as L
    from gpullama3_hip.model import CONFIGS, synth_model

    shape = CONFIGS[key].with_(context_length=n_prompt + n_gen)
    tensors = synth_model(shape, seed, norm_init="ones")
    prompt = np.random.default_rng(seed).integers(0, shape.vocab_size, n_prompt)
    out = {"workload": f"{key}: {shape.name}, {n_prompt}-token random prompt then {n_gen} greedy tokens from "
                       f"position 0", "prompt_tokens": n_prompt, "generated_tokens": n_gen}
    toks = {}
    runs = (("prefill", 0), ("stepwise", L.FLAG_STEPWISE_PROMPT)) if stepwise else (("prefill", 0),)
    for name, flags in runs:
        plan = HipMasterPlan.initialize_plan(shape, tensors, flags=flags)
        plan.generate_from_prompt(prompt, 0, 4)  # warm the path
        plan.reset()
        t1 = time.perf_counter()
        toks[name] = plan.generate_from_prompt(prompt, 0, n_gen)
        dt = time.perf_counter() - t1
        r = {"tok_s": round((n_prompt + n_gen) / dt, 2), "wall_ms": round(1e3 * dt, 3)}
        if name == "prefill":
            plan.reset()
            t1 = time.perf_counter()
            plan.prefill(prompt[:-1], 0)
            dp = time.perf_counter() - t1
            fl = prefill_flops(shape, n_prompt - 1)
            r.update({"prefill_ms": round(1e3 * dp, 3), "prefill_tok_s": round((n_prompt - 1) / dp, 1),
                      "prefill_tflops": round(fl / dp / 1e12, 2),
                      "prefill_mfma_frac": round(fl / dp / 2.5e15, 4),
                      "prefill_note": "algorithmic flops of the 511 prompt rows (matrix products and causal "
                                      "attention) / time, against 2.5 PFLOP/s dense fp16; the products issue "
                                      "twice the MFMA work (hi and lo fp16 parts of the activations)"})
        out[name] = r
        plan.free_execution_plan()
    if stepwise:
        out["tokens_equal"] = bool(np.array_equal(toks["prefill"], toks["stepwise"]))
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode steps of the headline workload (exact)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="llama1b_q8")
    ap.add_argument("--schedule", default="persistent", choices=["persistent", "graph"])
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--starts", default=None,
                    help="comma-separated segment start positions (KV history filled to each); default: the "
                         "configuration's spread of positions")
    ap.add_argument("--steps-8b", type=int, default=128, help="greedy steps at each 8B KV fill")
    ap.add_argument("--no-8b", action="store_true", help="leave out the Llama-3.1-8B part of the line")
    ap.add_argument("--no-prompt", action="store_true", help="leave out the Qwen3 prompt workload")
    ap.add_argument("--attention-only", action="store_true",
                    help="run only the standalone attention kernel of the Llama-3.1-8B shape at each KV fill and "
                         "print its JSON object")
    ap.add_argument("--prompt-only", default=None, metavar="CONFIG",
                    help="run only the prompt workload (512-token prompt through the batched prefill, then 256 "
                         "greedy tokens) on CONFIG and print its JSON object")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only the plain copy kernel used to calibrate rocprofv3 byte counters")
    ap.add_argument("--calibrate-first", action="store_true",
                    help="run the copy kernel in this process before the benchmark, so that one rocprofv3 --pmc "
                         "session holds both (the byte counters' scale differs between sessions)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this decode path has no multi-GPU mode (--gpus {args.gpus} refused)",
              file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.calibrate_first:
        copy_calibration(out=sys.stderr)

    from gpullama3_hip import device_name
    from gpullama3_hip import _lib as L

    if args.attention_only:
        print(json.dumps(attention_only(args.seed)), flush=True)
        return
    if args.prompt_only:
        print(json.dumps(prompt_workload(args.seed, key=args.prompt_only, stepwise=False)), flush=True)
        return

    starts = [int(v) for v in args.starts.split(",")] if args.starts else None
    log(f"device: {device_name()}")
    main_run = bench_config(args.config, args.steps, args.warmup, args.seed, args.schedule, starts)
    shape, plan, res = main_run["shape"], main_run["plan"], main_run["res"]
    log(f"{args.config}: {main_run['tok_s']:.1f} tok/s, {main_run['roofline']['achieved']} GB/s "
        f"({100 * main_run['roofline']['frac']:.1f}% of 8 TB/s)")
    ref_wl = None
    if args.schedule == "persistent" and shape.context_length >= 256:
        ref_wl = reference_workload(plan, shape, args.seed)
        log(f"reference workload (128 prompt + 128 greedy from position 0): {ref_wl['tok_s']} tok/s")
        ref_wl["sampled"] = reference_workload_sampled(plan, shape, args.seed)
        log(f"reference workload with the default top-p sampler: {ref_wl['sampled']['tok_s']} tok/s")
    plan.free_execution_plan()
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(shape, main_run["tensors"], [s for s, _ in main_run["segs"]])
        log(f"cpu baseline: {cpu}")
    del main_run["tensors"]

    part_8b = None
    if args.config == "llama1b_q8" and not args.no_8b and args.steps_8b > 0:
        r8 = bench_config("llama8b_q8", args.steps_8b * len(FILLS_8B), args.warmup, args.seed, args.schedule,
                          with_attention=args.schedule == "persistent")
        r8["plan"].free_execution_plan()
        cpu8 = None
        if not args.no_cpu_baseline:
            v8, n8, t8, b8 = cpu_decode_rate(r8["shape"], r8["tensors"], FILLS_8B, 2, cpu_threads())
            cpu8 = {"value": round(v8, 3), "unit": "tok/s", "threads": cpu_threads(), "kind": "port",
                    "sample": f"{n8} greedy steps, 2 from each fill {list(FILLS_8B)}, fp32 KV, {t8:.1f} s",
                    "achieved_gbs": round(b8 / t8 / 1e9, 2)}
        del r8["tensors"]
        part_8b = {"workload": f"llama8b_q8: {r8['shape'].name}, batch-1 greedy decode, {args.steps_8b} steps at "
                               f"each fp16 N(0,1) KV fill {list(FILLS_8B)}",
                   "value": round(r8["tok_s"], 2), "unit": "tok/s", "steps": r8["res"]["steps"],
                   "ms_per_step": round(1e3 * r8["res"]["wall_s"] / r8["res"]["steps"], 4),
                   "roofline": r8["roofline"], "segments": r8["res"]["segments"],
                   "attention_kernel": r8.get("attention"), "cpu_baseline": cpu8}
        log(f"llama8b_q8: {r8['tok_s']:.1f} tok/s, {r8['roofline']['achieved']} GB/s")

    prompt_wl = None
    if args.config == "llama1b_q8" and not args.no_prompt:
        prompt_wl = prompt_workload(args.seed)
        log(f"qwen3 prompt workload: {prompt_wl['prefill']['tok_s']} tok/s with the batched prefill "
            f"({prompt_wl['prefill']['prefill_ms']} ms for 511 prompt tokens), {prompt_wl['stepwise']['tok_s']} "
            f"tok/s stepwise")

    rec = {
        "metric": METRIC,
        "value": round(main_run["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": res["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * res["wall_s"] / res["steps"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 weights, fp32 accumulate" if shape.weight_type == L.TYPE_Q8_0 else "fp16 weights, fp32 accumulate",
        "data": "synthetic (seeded random-init weights, N(0,1) fp16 KV history)",
        "config": {"workload": f"{args.config}: {shape.name}, batch-1 greedy decode, {res['steps']} tokens in "
                               f"segments (start, tokens) {main_run['segs']}",
                   "layers": shape.n_layers, "dim": shape.dim, "vocab": shape.vocab_size,
                   "schedule": args.schedule},
        "achieved_hbm_gbs": main_run["roofline"]["achieved"],
        "hbm_fraction": main_run["roofline"]["frac"],
        "roofline": main_run["roofline"],
        "segments": res["segments"],
        "cpu_baseline": cpu,
        "reference_workload": ref_wl,
        "llama8b_q8": part_8b,
        "qwen3_prompt": prompt_wl,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
