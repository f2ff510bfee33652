"""Batched prefill (gl3_prefill, and the prompt phase of the generate calls)
against the oracle, which forwards the prompt one token at a time as the
reference does (InferenceEngine.java:88-131, :162-187).

Bars, with the oracle's test aids kv_fp16 (the device's fp16 rounding of K and
V) and f16_exact (FP16 weights decoded exactly, subnormals kept, as the device
does; the reference's vector path flushes them):
* the K and V the prefill leaves at every prompt position of every layer agree
  with the oracle's within 4e-3 of the layer's largest magnitude (fp16 values
  that differ by at most a unit in the last place, or by the fp32 summation
  order's effect before the rounding);
* the logits of the decode steps that follow (the last prompt token, then
  teacher-forced greedy tokens) agree within 2e-3 of their std, the decode
  step's own tight bar;
* the greedy tokens of gl3_generate_from_prompt equal the oracle's up to the
  first step whose top-2 margin is within the 2e-2 * std tolerance.
"""
import ctypes

import numpy as np
import pytest

import oracle.oracle as orc
from gpullama3_hip import _lib as L
from harness import build, check_kv, small, top2_margin

pytestmark = pytest.mark.gpu

TOL_TIGHT = 2e-3
TOL_REF = 2e-2

SCHEDULES = {"persistent": 0, "graph": L.FLAG_PHASE_KERNELS}


def teacher_forced(plan, ref, tok, pos, n, tol=TOL_TIGHT):
    """n decode steps from (tok, pos) on both sides, each feeding the oracle's argmax."""
    worst = 0.0
    for i in range(n):
        lg, am = plan.forward(int(tok), int(pos + i))
        rl = ref.forward(int(tok), int(pos + i))
        d = float(np.max(np.abs(lg - rl)) / rl.std())
        worst = max(worst, d)
        assert d <= tol, (pos + i, d)
        if top2_margin(rl) > tol * rl.std():
            assert am == orc.argmax(rl), (pos + i, am, orc.argmax(rl))
        tok = orc.argmax(rl)
    return worst


@pytest.mark.parametrize("key", ["llama1b_q8", "llama1b_f16", "qwen3_06b_q8", "phi3_mini_f16", "llama8b_q8",
                                 "llama3b_q8", "qwen3_4b_f16"])
def test_prefill_matches_oracle(gpu, key):
    """A ragged 77-token prompt: 76 tokens batched, then the last one and 4 greedy steps decoded."""
    shape = small(key, ctx=256)
    if key == "llama1b_f16":
        shape = shape.with_(tied=True)
    print(f"[case] {key} prefill 76 + decode 5", flush=True)
    plan, ref, _ = build(shape, kv_fp16=True, f16_exact=True)
    prompt = np.random.default_rng(21).integers(0, shape.vocab_size, 77)
    plan.prefill(prompt[:-1], 0)
    for i, t in enumerate(prompt[:-1]):
        ref.forward(int(t), i)
    kvd = check_kv(plan, ref, shape, 0, 76)
    d = teacher_forced(plan, ref, prompt[-1], 76, 5)
    print(f"  KV max|d|/max|ref| {kvd:.2e}; logits max|d|/std {d:.2e}", flush=True)
    plan.free_execution_plan()
    ref.close()


def test_prefill_blocks_after_decode(gpu):
    """40 decode steps, then a 600-token prefill from position 40 (two blocks of
    rows: 512 + 88), then decode again: the prefill reads history it did not
    write and the decode reads what the prefill wrote."""
    shape = small("llama1b_q8", ctx=768)
    print("[case] llama1b_q8 decode 40, prefill 600 at 40, decode 4", flush=True)
    plan, ref, _ = build(shape, kv_fp16=True)
    toks = np.random.default_rng(22).integers(0, shape.vocab_size, 641)
    for i in range(40):
        plan.forward(int(toks[i]), i, logits=False)
        ref.forward(int(toks[i]), i)
    plan.prefill(toks[40:640], 40)
    for i in range(40, 640):
        ref.forward(int(toks[i]), i)
    kvd = check_kv(plan, ref, shape, 0, 640)
    d = teacher_forced(plan, ref, toks[640], 640, 4)
    print(f"  KV max|d|/max|ref| {kvd:.2e}; logits max|d|/std {d:.2e}", flush=True)
    plan.free_execution_plan()
    ref.close()


def oracle_greedy(ref, prompt, n_gen):
    """The oracle's prompt phase and greedy steps; (tokens, margins / tolerance)."""
    for i, t in enumerate(prompt[:-1]):
        ref.forward(int(t), i)
    tok, out, ok = int(prompt[-1]), [], []
    for i in range(n_gen):
        rl = ref.forward(tok, len(prompt) - 1 + i)
        tok = orc.argmax(rl)
        out.append(tok)
        ok.append(top2_margin(rl) > TOL_REF * rl.std())
    return np.array(out), ok


def agree_until_tie(got, want, ok):
    for i in range(len(want)):
        assert got[i] == want[i], (i, got[:i + 1], want[:i + 1])
        if not ok[i]:  # a near tie: later tokens may follow either branch
            return i + 1
    return len(want)


@pytest.mark.parametrize("sched", sorted(SCHEDULES))
def test_generate_from_prompt_with_prefill(gpu, sched):
    shape = small("qwen3_06b_q8", ctx=256)
    print(f"[case] qwen3 generate_from_prompt 100 + 24, {sched}", flush=True)
    plan, ref, tensors = build(shape, flags=SCHEDULES[sched], kv_fp16=False)
    prompt = np.random.default_rng(23).integers(0, shape.vocab_size, 100)
    want, ok = oracle_greedy(ref, prompt, 24)
    got = plan.generate_from_prompt(prompt, 0, 24)
    n = agree_until_tie(got, want, ok)
    print(f"  {n} tokens equal to the oracle's", flush=True)
    # the same call with the prompt forwarded one decode step per token
    from gpullama3_hip import HipMasterPlan
    step = HipMasterPlan.initialize_plan(shape, tensors, flags=SCHEDULES[sched] | L.FLAG_STEPWISE_PROMPT)
    got2 = step.generate_from_prompt(prompt, 0, 24)
    agree_until_tie(got2, want, ok)
    # sampling at temperature 0 takes the same path and the same tokens
    plan.reset()
    got3 = plan.generate_sampled(prompt, 0, 24, 0.0, 0.95, np.zeros(24, np.float32))
    assert np.array_equal(got3, got)
    step.free_execution_plan()
    plan.free_execution_plan()
    ref.close()


def test_prefill_rejects_bad_arguments(gpu):
    shape = small("llama1b_q8", ctx=128)
    plan, ref, _ = build(shape)
    lib = plan.lib
    toks = np.arange(10, dtype=np.int32)
    ip = toks.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    assert lib.gl3_prefill(plan.h, ip, 0, 0) == L.ERR_INVALID_ARGUMENT
    assert lib.gl3_prefill(plan.h, ip, 10, 119) == L.ERR_INVALID_ARGUMENT  # past the context
    assert lib.gl3_prefill(plan.h, ip, 10, -1) == L.ERR_INVALID_ARGUMENT
    assert lib.gl3_prefill(plan.h, None, 10, 0) == L.ERR_INVALID_ARGUMENT
    assert lib.gl3_prefill(None, ip, 10, 0) == L.ERR_INVALID_ARGUMENT
    bad = toks.copy()
    bad[3] = shape.vocab_size
    assert lib.gl3_prefill(plan.h, bad.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), 10, 0) == \
        L.ERR_INVALID_ARGUMENT
    assert b"out of range" in lib.gl3_last_error()
    # still usable, and the full context can be filled
    plan.prefill(np.arange(128) % shape.vocab_size, 0)
    plan.free_execution_plan()
    ref.close()
