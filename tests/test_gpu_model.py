"""End-to-end parity of the decode step against the oracle, through the C ABI.

Two bars: against the oracle with the test aid kv_fp16 (same fp16 KV rounding
as the device) logits agree to 2e-3 of their std; against the oracle with the
reference's own fp32 KV cache they agree within the 2e-2 * std tolerance and
greedy tokens match wherever the top-2 margin exceeds it.  Both schedules (the
persistent per-token kernel and the per-phase hipGraph) are checked.
"""
import numpy as np
import pytest

import oracle.oracle as orc
from gpullama3_hip import HipMasterPlan
from gpullama3_hip import _lib as L
from gpullama3_hip.gguf import write_gguf
from gpullama3_hip.model import synth_model
from harness import build, prefill_from_device, prefill_kv, small, top2_margin

pytestmark = pytest.mark.gpu

TOL_REF = 2e-2     # parity bar against the reference's CPU forward: max |d logits| / std(logits)
TOL_TIGHT = 2e-3   # same arithmetic up to fp32 summation order (10x inside TOL_REF)

SCHEDULES = {"persistent": 0, "graph": L.FLAG_PHASE_KERNELS}


def run_steps(plan, ref, toks, poss):
    out = []
    for t, p in zip(toks, poss):
        lg, am = plan.forward(int(t), int(p))
        rl = ref.forward(int(t), int(p))
        out.append((lg, am, rl))
    return out


@pytest.mark.parametrize("sched", sorted(SCHEDULES))
@pytest.mark.parametrize("key", ["llama1b_q8", "qwen3_06b_q8", "llama1b_f16", "phi3_mini_f16", "llama8b_q8",
                                 "llama3b_q8", "qwen3_4b_f16", "phi3_mini_q8", "mistral7b_f16"])
def test_decode_matches_oracle(gpu, key, sched):
    shape = small(key)
    if key == "llama1b_f16":
        shape = shape.with_(tied=True)
    print(f"[case] {key} {sched} shape={shape}", flush=True)
    plan, ref, _ = build(shape, flags=SCHEDULES[sched], kv_fp16=True)
    rng = np.random.default_rng(11)
    prefill = 130  # > two attention splits of 64 positions
    prefill_kv(plan, ref, shape, prefill)
    toks = rng.integers(0, shape.vocab_size, 6)
    poss = np.arange(prefill, prefill + 6)
    for lg, am, rl in run_steps(plan, ref, toks, poss):
        d = np.max(np.abs(lg - rl)) / rl.std()
        print(f"  max|d|/std = {d:.2e}", flush=True)
        assert d <= TOL_TIGHT, d
        assert am == int(np.argmax(lg))
        if top2_margin(rl) > TOL_TIGHT * rl.std():
            assert am == orc.argmax(rl)
    plan.free_execution_plan()
    ref.close()


@pytest.mark.parametrize("sched", sorted(SCHEDULES))
def test_two_tile_attention_ring_at_long_context(gpu, sched):
    """Qwen3-4B FP16, whose persistent kernel keeps two K/V tiles in flight per
    wave: positions past 7000, where a split spans four tiles per wave (the
    waits then count one tile issued ahead), against the oracle."""
    shape = small("qwen3_4b_f16", ctx=8192)
    print(f"[case] qwen3_4b_f16 {sched} at 7000+", flush=True)
    plan, ref, _ = build(shape, flags=SCHEDULES[sched], kv_fp16=True)
    prefill_from_device(plan, ref, shape, 7000)
    rng = np.random.default_rng(13)
    toks = rng.integers(0, shape.vocab_size, 3)
    for lg, am, rl in run_steps(plan, ref, toks, np.arange(7000, 7003)):
        d = np.max(np.abs(lg - rl)) / rl.std()
        print(f"  max|d|/std = {d:.2e}", flush=True)
        assert d <= TOL_TIGHT, d
        if top2_margin(rl) > TOL_TIGHT * rl.std():
            assert am == orc.argmax(rl)
    plan.free_execution_plan()
    ref.close()


def test_attention_split_count_switch(gpu):
    """The fused-FFN shape halves its attention splits once a split would pass
    48 positions (1536 positions with 32 splits of a kv head): decode steps across
    the switch against the oracle."""
    shape = small("llama1b_q8", ctx=2048)
    print("[case] llama1b_q8 split switch at 1536", flush=True)
    plan, ref, _ = build(shape, kv_fp16=True)
    prefill_from_device(plan, ref, shape, 1532)
    rng = np.random.default_rng(17)
    toks = rng.integers(0, shape.vocab_size, 8)
    for lg, am, rl in run_steps(plan, ref, toks, np.arange(1532, 1540)):
        d = np.max(np.abs(lg - rl)) / rl.std()
        print(f"  max|d|/std = {d:.2e}", flush=True)
        assert d <= TOL_TIGHT, d
        if top2_margin(rl) > TOL_TIGHT * rl.std():
            assert am == orc.argmax(rl)
    plan.free_execution_plan()
    ref.close()


@pytest.mark.parametrize("key", ["llama1b_q8", "qwen3_06b_q8"])
def test_decode_vs_reference_fp32_kv(gpu, key):
    shape = small(key)
    plan, ref, _ = build(shape, kv_fp16=False)
    rng = np.random.default_rng(5)
    toks = rng.integers(0, shape.vocab_size, 20)
    for lg, am, rl in run_steps(plan, ref, toks, np.arange(20)):
        tol = TOL_REF * rl.std()
        assert np.max(np.abs(lg - rl)) <= tol
        if top2_margin(rl) > tol:
            assert am == orc.argmax(rl)
    plan.free_execution_plan()


@pytest.mark.parametrize("sched", sorted(SCHEDULES))
def test_generate_greedy_matches_stepwise(gpu, sched):
    shape = small("llama1b_q8")
    plan, ref, _ = build(shape, flags=SCHEDULES[sched])
    gen = plan.generate_greedy(17, 0, 24)
    plan.reset()
    tok, step = 17, []
    for p in range(24):
        _, tok = plan.forward(tok, p)
        step.append(tok)
    assert list(gen) == step
    # the oracle's greedy run agrees while its top-2 margin allows
    ref.reset()
    tok = 17
    for p in range(24):
        rl = ref.forward(tok, p)
        if top2_margin(rl) <= TOL_TIGHT * rl.std():
            break
        assert orc.argmax(rl) == gen[p]
        tok = gen[p]
    plan.free_execution_plan()


def test_generate_greedy_across_launches(gpu):
    """The persistent schedule decodes up to 256 tokens per launch; a run of
    300 spans two launches and must repeat the per-token forwards exactly."""
    shape = small("llama1b_q8", ctx=320)
    plan, ref, _ = build(shape)
    ref.close()
    gen = plan.generate_greedy(3, 10, 300)
    plan.reset()
    tok = 3
    for i in range(300):
        _, tok = plan.forward(tok, 10 + i)
        assert tok == gen[i], i
    plan.free_execution_plan()


@pytest.mark.parametrize("sched", sorted(SCHEDULES))
@pytest.mark.parametrize("key", ["llama1b_q8", "llama8b_q8"])
def test_upload_after_forward_replaces_ffn_weights(gpu, key, sched):
    """Weights uploaded after a forward are what the next forward uses, also
    where the persistent kernel keeps a rearranged copy of an FFN matrix (the
    sliced Wdown of the fused FFN of the 1B Q8_0 shape) and where the per-phase
    schedule captured a graph."""
    shape = small(key)
    plan, ref, tensors = build(shape, flags=SCHEDULES[sched])
    ref.close()
    plan.forward(5, 0)
    other = synth_model(shape, seed=99)
    for name in ("blk.0.ffn_gate.weight", "blk.0.ffn_up.weight", "blk.1.ffn_down.weight"):
        tensors[name] = other[name]
        plan.upload(name, other[name][0].ggml_type, other[name][1])
    plan.reset()
    ref = orc.OracleModel(shape, tensors, kv_fp16=True)
    for p, t in enumerate([5, 99, 7]):
        lg, am = plan.forward(t, p)
        rl = ref.forward(t, p)
        assert np.max(np.abs(lg - rl)) <= TOL_TIGHT * rl.std()
    plan.free_execution_plan()
    ref.close()


@pytest.mark.parametrize("sched", sorted(SCHEDULES))
def test_output_weight_uploaded_to_tied_plan(gpu, sched):
    """A tied plan (no output.weight: the classifier is token_embd) that receives
    an output.weight after its first forward uses it from then on, on both
    schedules (the per-phase graph is captured again)."""
    shape = small("llama1b_f16").with_(tied=True)
    plan, ref, tensors = build(shape, flags=SCHEDULES[sched])
    lg0, _ = plan.forward(5, 0)
    assert np.max(np.abs(lg0 - ref.forward(5, 0))) <= TOL_TIGHT * lg0.std()
    ref.close()
    from gpullama3_hip.model import F16, TensorSpec, synth_tensor
    spec = TensorSpec("output.weight", F16, shape.vocab_size, shape.dim)
    tensors["output.weight"] = (spec, synth_tensor(spec, 99))
    plan.upload("output.weight", F16, tensors["output.weight"][1])
    plan.reset()
    ref = orc.OracleModel(shape, tensors, kv_fp16=True)
    for p, t in enumerate([5, 99, 7]):
        lg, am = plan.forward(t, p)
        rl = ref.forward(t, p)
        assert np.max(np.abs(lg - rl)) <= TOL_TIGHT * rl.std(), p
    plan.free_execution_plan()
    ref.close()


def test_plan_lifecycle_releases_device_memory(gpu):
    """create / upload / forward / destroy returns every device allocation,
    including the Q8_0 upload staging buffer (hipMemGetInfo before and after)."""
    import ctypes
    # the HIP runtime the library already loaded (not a second copy)
    with open("/proc/self/maps") as f:
        paths = sorted({ln.split()[-1] for ln in f if "libamdhip64.so" in ln})
    assert paths, "libamdhip64 is not loaded"
    hip = ctypes.CDLL(paths[0])
    free, total = ctypes.c_size_t(), ctypes.c_size_t()

    def free_bytes():
        assert hip.hipDeviceSynchronize() == 0
        assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
        return free.value

    # a 64k-row Q8_0 classifier: a 139 MB staging buffer per plan if it leaked
    shape = small("llama1b_q8", vocab=65536)
    tensors = synth_model(shape, 7, norm_init="random")

    def cycle():
        plan = HipMasterPlan.initialize_plan(shape, tensors)
        plan.forward(3, 0)
        plan.free_execution_plan()

    cycle()  # runtime pools and code objects
    f0 = free_bytes()
    for _ in range(3):
        cycle()
    f1 = free_bytes()
    print(f"device memory free before {f0 >> 20} MiB, after 3 cycles {f1 >> 20} MiB", flush=True)
    assert f1 >= f0 - (32 << 20)


@pytest.mark.parametrize("sched", sorted(SCHEDULES))
def test_gqa8_decode_matches_oracle(gpu, sched):
    """GQA group 8 (32 query heads over 4 kv heads): no compiled persistent shape,
    so both flags run the per-phase schedule; against the oracle over a history
    longer than two attention splits."""
    shape = small("llama1b_q8").with_(n_kv_heads=4)
    print(f"[case] GQA 8 {sched} shape={shape}", flush=True)
    plan, ref, _ = build(shape, flags=SCHEDULES[sched], kv_fp16=True)
    prefill_kv(plan, ref, shape, 130)
    rng = np.random.default_rng(21)
    toks = rng.integers(0, shape.vocab_size, 4)
    for lg, am, rl in run_steps(plan, ref, toks, np.arange(130, 134)):
        assert np.max(np.abs(lg - rl)) <= TOL_TIGHT * rl.std()
        if top2_margin(rl) > TOL_TIGHT * rl.std():
            assert am == orc.argmax(rl)
    plan.free_execution_plan()
    ref.close()


def test_schedules_agree_and_are_deterministic(gpu):
    shape = small("llama1b_q8")
    a, ref, tensors = build(shape, flags=0)
    b, _, _ = build(shape, flags=L.FLAG_PHASE_KERNELS)
    for p, t in enumerate([5, 99, 1234, 7]):
        la, _ = a.forward(t, p)
        lb, _ = b.forward(t, p)
        assert np.max(np.abs(la - lb)) <= TOL_TIGHT * la.std()
    a.reset()
    l1 = [a.forward(t, p)[0] for p, t in enumerate([5, 99])]
    a.reset()
    l2 = [a.forward(t, p)[0] for p, t in enumerate([5, 99])]
    for x, y in zip(l1, l2):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


def test_kv_cache_holds_rotated_keys(gpu):
    shape = small("qwen3_06b_q8")
    plan, ref, _ = build(shape)
    for p, t in enumerate([3, 4, 5]):
        plan.forward(t, p)
        ref.forward(t, p)
    for l in range(shape.n_layers):
        k, v = plan.read_kv(l, 0, 3)
        rk, rv = ref.kv(l)
        assert np.allclose(k.view(np.float16).astype(np.float32), rk[:3], rtol=2e-3, atol=1e-3)
        assert np.allclose(v.view(np.float16).astype(np.float32), rv[:3], rtol=2e-3, atol=1e-3)


def test_forward_argument_errors(gpu):
    shape = small("llama1b_q8")
    plan, _, _ = build(shape)
    with pytest.raises(ValueError):
        plan.forward(shape.vocab_size, 0)
    with pytest.raises(ValueError):
        plan.forward(0, shape.context_length)
    with pytest.raises(ValueError):
        plan.generate_greedy(0, shape.context_length - 2, 5)


def test_phase_trace_is_ordered(gpu):
    """Phase stamps of the persistent kernel (GL3_FLAG_PHASE_TRACE): one row per
    boundary, every workgroup's stamps advance through the token, and a traced
    run decodes the same tokens as an untraced one."""
    shape = small("llama1b_q8")
    plan, ref, tensors = build(shape, flags=L.FLAG_PHASE_TRACE)
    gen = plan.generate_greedy(17, 0, 6)
    st = plan.phase_stamps().astype(np.int64)
    assert st.shape[0] == 3 + 10 * shape.n_layers + 1
    assert (np.diff(st, axis=0) >= 0).all()
    tr = plan.phase_trace()
    assert len(tr) == st.shape[0] - 1 and (tr >= 0).all()
    plain = HipMasterPlan.initialize_plan(shape, tensors)
    assert np.array_equal(plain.generate_greedy(17, 0, 6), gen)
    plain.free_execution_plan()
    plan.free_execution_plan()
    ref.close()


@pytest.mark.parametrize("key", ["llama1b_q8", "llama1b_f16", "qwen3_06b_q8", "phi3_mini_f16"])
def test_plan_from_gguf_matches_upload(gpu, tmp_path, key):
    """gl3_create_from_gguf (the library parses the file, maps it and uploads from
    the mapping) gives bit-identical logits to uploading the same tensors."""
    shape = small(key)
    if key == "llama1b_f16":
        shape = shape.with_(tied=True)
    print(f"[case] {key} from GGUF", flush=True)
    tensors = synth_model(shape, 7, norm_init="random")
    path = tmp_path / "m.gguf"
    write_gguf(path, shape, tensors)
    a = HipMasterPlan.initialize_plan(shape, tensors)
    b = HipMasterPlan.from_gguf(path, shape.context_length)
    # the oracle with the device's exact fp16 decode: the tight bar compares the same arithmetic
    ref = orc.OracleModel(shape, tensors, kv_fp16=True, f16_exact=True)
    assert b.shape.vocab_size == shape.vocab_size and b.shape.n_layers == shape.n_layers
    for pos, tok in enumerate([3, 1000, 77, 4095]):
        la, ta = a.forward(tok, pos)
        lb, tb = b.forward(tok, pos)
        assert np.array_equal(la, lb) and ta == tb, pos
        # the file-loaded plan against the oracle fed the tensors the file was written from
        rl = ref.forward(tok, pos)
        assert np.max(np.abs(lb - rl)) <= TOL_TIGHT * rl.std(), pos
        if top2_margin(rl) > TOL_TIGHT * rl.std():
            assert tb == orc.argmax(rl)
    a.free_execution_plan()
    b.free_execution_plan()
    ref.close()


@pytest.mark.parametrize("sched", sorted(SCHEDULES))
@pytest.mark.parametrize("n_prompt,n_gen", [(1, 5), (37, 20), (200, 99)])
def test_generate_from_prompt_matches_stepwise(gpu, sched, n_prompt, n_gen):
    """Prompt forced then greedy on the device (one call; 200 + 99 - 1 steps cross a
    launch boundary) equals the same loop driven token by token from the host."""
    shape = small("llama1b_q8")
    plan, ref, _ = build(shape, flags=SCHEDULES[sched])
    prompt = np.random.default_rng(4).integers(0, shape.vocab_size, n_prompt)
    start = 3
    gen = plan.generate_from_prompt(prompt, start, n_gen)
    plan.reset()
    am = None
    for i, t in enumerate(prompt):
        _, am = plan.forward(int(t), start + i)
    toks = [am]
    for j in range(n_gen - 1):
        _, am = plan.forward(toks[-1], start + n_prompt + j)
        toks.append(am)
    assert list(gen) == toks
    plan.free_execution_plan()
    ref.close()


def test_generate_from_prompt_argument_errors(gpu):
    shape = small("llama1b_q8")
    plan, ref, _ = build(shape)
    with pytest.raises(ValueError):
        plan.generate_from_prompt([1, shape.vocab_size], 0, 4)
    with pytest.raises(ValueError):
        plan.generate_from_prompt([1, 2, 3], shape.context_length - 4, 3)
    with pytest.raises(ValueError):
        plan.generate_from_prompt([], 0, 3)
    assert len(plan.generate_from_prompt([1, 2, 3], shape.context_length - 5, 3)) == 3
    plan.free_execution_plan()
    ref.close()
