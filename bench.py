"""Decode throughput benchmark (one MI355X).

Default workload: Llama-3.2-1B-shaped model with Q8_0 linear weights (FP16
embeddings), batch-1 greedy decode of 256 tokens spread over positions 0-2048
(8 segments of 32 steps; before each segment the fp16 KV cache holds N(0,1)
history up to the segment's start).  Weights are random-init from a seed (no
checkpoints).  One JSON line on stdout; details on stderr.

    python bench.py [--steps 256] [--warmup 8] [--config llama1b_q8] [--schedule persistent|graph]
                    [--starts P1,P2,...]
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


def kv_bytes(shape, pos):
    """fp16 K and V of positions 0..pos, all layers."""
    return 2 * shape.n_layers * shape.kv_dim * 2 * (pos + 1)


def segments(cfg_key, steps, ctx, starts=None):
    if starts:
        per = max(1, steps // len(starts))
        return [(p, per) for p in starts]
    if cfg_key == "llama8b_q8":
        per = max(1, steps // 3)
        return [(p, per) for p in (8192, 16384, 32768)]
    nseg = 8 if steps >= 8 else 1
    per = steps // nseg
    span = 2048 if cfg_key.startswith("llama1b") else min(ctx, 4096) - per
    starts = [int(s) for s in np.linspace(0, max(0, span - per), nseg)]
    return [(s, per) for s in starts]


def cpu_baseline(shape, tensors, seconds=15.0):
    """The oracle (C restatement of the reference CPU forward, OpenMP over rows
    and heads) on this host's cores: decode from position 0 until ~`seconds`."""
    import oracle.oracle as orc
    threads = min(16, os.cpu_count() or 1)
    m = orc.OracleModel(shape, tensors, n_threads=threads)
    m.forward(1, 0)  # warm caches / thread pool
    m.reset()
    n, t0 = 0, time.perf_counter()
    tok = 1
    while time.perf_counter() - t0 < seconds and n < min(1024, shape.context_length):
        lg = m.forward(tok, n)
        tok = int(np.argmax(lg))
        n += 1
    dt = time.perf_counter() - t0
    m.close()
    return {"value": n / dt, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} greedy decode steps at positions 0-{n - 1} of the same model, oracle (C, OpenMP, "
                      f"AVX2 8-lane dots), {dt:.1f} s"}


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


def measured_traffic(cfg_key, tokens_per_launch):
    """HBM bytes per launch of the decode kernel from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration),
    rescaled from the profiled launch's token count to `tokens_per_launch`, or None."""
    path = os.path.join(ROOT, "profiles", f"traffic_decode_step_{cfg_key}.txt")
    if not os.path.exists(path):
        return None
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
        return None
    return int(per_token * tokens_per_launch)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed decode steps (default 256; llama8b_q8: 384, i.e. 128 at each of its three fills)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="llama1b_q8")
    ap.add_argument("--schedule", default="persistent", choices=["persistent", "graph"])
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--starts", default=None,
                    help="comma-separated segment start positions (KV history filled to each); default: the "
                         "configuration's spread of positions")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only the plain copy kernel used to calibrate rocprofv3 byte counters")
    ap.add_argument("--calibrate-first", action="store_true",
                    help="run the copy kernel in this process before the benchmark, so that one rocprofv3 --pmc "
                         "session holds both (the byte counters' scale differs between sessions)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.calibrate_first:
        copy_calibration(out=sys.stderr)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this decode path has no multi-GPU mode (--gpus {args.gpus} refused)",
              file=sys.stderr)
        sys.exit(2)

    from gpullama3_hip import HipMasterPlan, device_name
    from gpullama3_hip import _lib as L
    from gpullama3_hip.model import CONFIGS, synth_model, tensor_specs

    shape = CONFIGS[args.config]
    if args.steps is None:
        args.steps = 384 if args.config == "llama8b_q8" else 256
    log(f"device: {device_name()}  config: {args.config} {shape}")
    t0 = time.perf_counter()
    tensors = synth_model(shape, args.seed, norm_init="ones")
    log(f"synthetic weights: {time.perf_counter() - t0:.1f} s")
    flags = L.FLAG_TIMING | (L.FLAG_PHASE_KERNELS if args.schedule == "graph" else 0)
    plan = HipMasterPlan.initialize_plan(shape, tensors, flags=flags)
    wbytes = weight_bytes(shape, tensor_specs(shape))

    # warmup (untimed)
    if args.warmup > 0:
        plan.generate_greedy(1, 0, args.warmup)

    starts = [int(v) for v in args.starts.split(",")] if args.starts else None
    segs = segments(args.config, args.steps, shape.context_length, starts)
    if any(s < 0 or s + n > shape.context_length for s, n in segs):
        print(f"segments {segs} do not fit the context of {shape.context_length} positions", file=sys.stderr)
        sys.exit(2)
    total_steps = sum(n for _, n in segs)
    wall = 0.0
    kern_ms = 0.0
    launches = 0
    algo_bytes = 0.0
    tok = 1
    for start, n in segs:
        plan.reset()
        if start > 0:
            plan.fill_kv_normal(args.seed + start, start)
        t1 = time.perf_counter()
        out = plan.generate_greedy(tok, start, n)
        t2 = time.perf_counter()
        el, km, nl = plan.timing()
        wall += t2 - t1
        kern_ms += km
        launches += nl
        seg_bytes = sum(wbytes + kv_bytes(shape, start + i) for i in range(n))
        algo_bytes += seg_bytes
        log(f"segment start={start:6d} steps={n}: wall {1e3 * (t2 - t1) / n:.3f} ms/token, "
            f"stream {el / n:.3f} ms/token, kernel {km / n:.3f} ms/token over {nl} launch(es), "
            f"{seg_bytes / (km * 1e-3) / 1e9:.0f} GB/s algorithmic")
        tok = int(out[-1])
    tok_s = total_steps / wall
    # the reference's own workload shape and count: a 128-token random prompt, then
    # 128 greedy tokens from position 0, tokens/s = (prompt + generated) / wall time
    # (InferenceEngine.java:134-138); prompt and generation both on the device
    ref_wl = None
    if args.schedule == "persistent" and shape.context_length >= 256:
        plan.reset()
        prompt = np.random.default_rng(args.seed).integers(0, shape.vocab_size, 128)
        plan.generate_from_prompt(prompt, 0, 4)  # warm the path
        plan.reset()
        t1 = time.perf_counter()
        plan.generate_from_prompt(prompt, 0, 128)
        t2 = time.perf_counter()
        ref_wl = {"prompt_tokens": 128, "generated_tokens": 128, "tok_s": round(256 / (t2 - t1), 2),
                  "wall_ms": round(1e3 * (t2 - t1), 3),
                  "note": "(prompt + generated) / wall time from position 0, as the reference counts its tok/s"}
        log(f"reference workload (128 prompt + 128 greedy from position 0): {ref_wl['tok_s']} tok/s")
    # one persistent launch decodes a whole segment; per-launch figures are
    # averages over the timed launches
    avg_kernel_s = kern_ms * 1e-3 / launches
    avg_bytes = algo_bytes / launches
    achieved = avg_bytes / avg_kernel_s / 1e9
    plan.free_execution_plan()

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(shape, tensors)
        log(f"cpu baseline: {cpu}")

    kernel = (f"decode_step_kernel (one launch per segment of {total_steps // launches} tokens)"
              if args.schedule == "persistent" else "hipGraph of phase kernels (one replay per token)")
    rec = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": total_steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * wall / total_steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 weights, fp32 accumulate" if shape.weight_type == L.TYPE_Q8_0 else "fp16 weights, fp32 accumulate",
        "data": "synthetic (seeded random-init weights, N(0,1) fp16 KV history)",
        "config": {"workload": f"{args.config}: {shape.name}, batch-1 greedy decode, "
                               f"{total_steps} tokens at start positions {[s for s, _ in segs]}",
                   "layers": shape.n_layers, "dim": shape.dim, "vocab": shape.vocab_size,
                   "schedule": args.schedule},
        "achieved_hbm_gbs": round(achieved, 1),
        "hbm_fraction": round(achieved / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(args.config, total_steps / launches)
                     if args.schedule == "persistent" else None,
                     "kernel": kernel, "bytes_per_launch": int(avg_bytes),
                     "avg_launch_ms": round(avg_kernel_s * 1e3, 4)},
        "cpu_baseline": cpu,
        "reference_workload": ref_wl,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
