"""Shared helpers: build the device plan and the oracle from the same tensors."""
import numpy as np

import oracle.oracle as orc
from gpullama3_hip import HipMasterPlan
from gpullama3_hip.model import CONFIGS, synth_model

# Per-layer shapes of the five workloads (with few layers and a small vocabulary
# they keep the compile-time GEMV shapes of the persistent kernel).
LAYER_SHAPES = {
    "llama1b_q8": CONFIGS["llama1b_q8"],
    "llama1b_f16": CONFIGS["llama1b_f16"],
    "qwen3_06b_q8": CONFIGS["qwen3_06b_q8"],
    "phi3_mini_f16": CONFIGS["phi3_mini_f16"],
    "llama8b_q8": CONFIGS["llama8b_q8"],
    "llama3b_q8": CONFIGS["llama3b_q8"],
    "qwen3_4b_f16": CONFIGS["qwen3_4b_f16"],
    "phi3_mini_q8": CONFIGS["phi3_mini_q8"],
    "mistral7b_f16": CONFIGS["mistral7b_f16"],
}


def small(key, n_layers=2, vocab=4096, ctx=512):
    return LAYER_SHAPES[key].with_(n_layers=n_layers, vocab_size=vocab, context_length=ctx)


def build(shape, seed=7, flags=0, norm_init="random", kv_fp16=True, threads=0, f16_exact=False):
    tensors = synth_model(shape, seed, norm_init=norm_init)
    plan = HipMasterPlan.initialize_plan(shape, tensors, flags=flags)
    ref = orc.OracleModel(shape, tensors, kv_fp16=kv_fp16, f16_exact=f16_exact, n_threads=threads)
    return plan, ref, tensors


def prefill_kv(plan, ref, shape, npos, seed=3):
    """Same fp16 N(0,1) history in both caches for positions [0, npos)."""
    rng = np.random.default_rng(seed)
    for l in range(shape.n_layers):
        k = rng.standard_normal((npos, shape.kv_dim), dtype=np.float32).astype(np.float16)
        v = rng.standard_normal((npos, shape.kv_dim), dtype=np.float32).astype(np.float16)
        plan.write_kv(l, 0, k.view(np.uint16), v.view(np.uint16))
        rk, rv = ref.kv(l)
        rk[:npos] = k.astype(np.float32)
        rv[:npos] = v.astype(np.float32)


def top2_margin(logits):
    s = np.sort(logits)
    return float(s[-1] - s[-2])


def prefill_from_device(plan, ref, shape, npos, seed=3):
    """The device's counter-based fp16 N(0,1) history (gl3_fill_kv_normal) for
    positions [0, npos), read back (gl3_read_kv) into the oracle's fp32 cache:
    both sides hold the same fp16-representable values.  Fast at long contexts."""
    plan.fill_kv_normal(seed, npos)
    for l in range(shape.n_layers):
        k, v = plan.read_kv(l, 0, npos)
        rk, rv = ref.kv(l)
        rk[:npos] = k.view(np.float16)
        rv[:npos] = v.view(np.float16)


TOL_KV = 4e-3  # K/V of a prefill: max |d| over the layer's largest magnitude


def check_kv(plan, ref, shape, pos0, npos):
    """Device K/V at [pos0, pos0 + npos) of every layer against the oracle's."""
    worst = 0.0
    for l in range(shape.n_layers):
        k, v = plan.read_kv(l, pos0, npos)
        rk, rv = ref.kv(l)
        for dev, want, what in ((k, rk, "K"), (v, rv, "V")):
            got = dev.view(np.float16).astype(np.float32)
            exp = want[pos0:pos0 + npos]
            scale = float(np.max(np.abs(exp)))
            d = np.abs(got - exp)
            rel = float(d.max()) / scale
            worst = max(worst, rel)
            if rel > TOL_KV:
                p, c = np.unravel_index(int(np.argmax(d)), d.shape)
                raise AssertionError(f"layer {l} {what} position {pos0 + p} column {c}: {got[p, c]} vs "
                                     f"{exp[p, c]} (max |d| / max |ref| = {rel:.2e})")
    return worst
