"""The benchmark's algorithmic byte count and workload layout (no GPU).

B(pos) = linear weight bytes (Q8_0 34/32 B, FP16 2 B per element, classifier
included) + fp16 K and V of positions 0..pos over all layers + one embedding
row.  The weight totals below are computed independently from the model shapes
(rows x cols per matrix); a dropped matrix, a wrong Q8_0 block size or a
missing classifier changes them.
"""
import pytest

import bench
from gpullama3_hip.model import CONFIGS, tensor_specs

Q8, F16 = 34 / 32, 2


def linear_bytes(dim, hidden, layers, q_dim, kv_dim, vocab, b, cls_b):
    per_layer = (q_dim + 2 * kv_dim) * dim + dim * q_dim + 2 * hidden * dim + dim * hidden
    return int(layers * per_layer * b + vocab * dim * cls_b)


EXPECTED = {  # linear weights per token, by hand from the shapes
    "llama1b_f16": linear_bytes(2048, 8192, 16, 2048, 512, 128256, F16, F16),
    "llama1b_q8": linear_bytes(2048, 8192, 16, 2048, 512, 128256, Q8, Q8),
    "qwen3_06b_q8": linear_bytes(1024, 3072, 28, 2048, 1024, 151936, Q8, Q8),
    "phi3_mini_f16": linear_bytes(3072, 8192, 32, 3072, 3072, 32064, F16, F16),
    "llama8b_q8": linear_bytes(4096, 14336, 32, 4096, 1024, 128256, Q8, Q8),
}


def test_weight_bytes_per_token():
    for key, want in EXPECTED.items():
        s = CONFIGS[key]
        assert bench.weight_bytes(s, tensor_specs(s)) == want + s.dim * 2, key  # + one embedding row


def test_published_table_values():
    # the per-token weight bytes of the five configurations as tabulated for the roofline targets
    assert EXPECTED["llama1b_q8"] == 1_312_980_992
    assert EXPECTED["llama1b_f16"] == 2_471_493_632
    assert EXPECTED["qwen3_06b_q8"] == 633_233_408
    assert EXPECTED["phi3_mini_f16"] == 7_444_758_528
    assert EXPECTED["llama8b_q8"] == 7_973_699_584


def test_kv_bytes():
    for key, per_pos in (("llama1b_q8", 32768), ("qwen3_06b_q8", 114688), ("phi3_mini_f16", 393216),
                         ("llama8b_q8", 131072)):
        s = CONFIGS[key]
        assert bench.kv_bytes(s, 0) == per_pos and bench.kv_bytes(s, 99) == 100 * per_pos


def test_segments_fit_the_workloads():
    s = CONFIGS["llama1b_q8"]
    segs = bench.segments("llama1b_q8", 256, s.context_length)
    assert len(segs) == 8 and all(n == 32 for _, n in segs)
    assert segs[0][0] == 0 and segs[-1][0] + 32 == 2048
    s8 = CONFIGS["llama8b_q8"]
    assert bench.segments("llama8b_q8", 384, s8.context_length) == [(8192, 128), (16384, 128), (32768, 128)]
    assert 32768 + 128 <= s8.context_length
    assert bench.segments("llama1b_q8", 64, s.context_length, [1024]) == [(1024, 64)]


@pytest.mark.parametrize("steps", [1, 5, 20, 31, 32, 33, 64, 100, 255, 256, 257, 300, 1000])
def test_segments_time_exactly_the_requested_steps(steps):
    """--steps K times K tokens (no truncation); launches keep >= 32 tokens when K allows,
    and the segments stay inside positions 0-2047 with their mean near the middle."""
    s = CONFIGS["llama1b_q8"]
    segs = bench.segments("llama1b_q8", steps, s.context_length)
    assert sum(n for _, n in segs) == steps
    assert all(n >= min(32, steps) for _, n in segs)
    assert all(0 <= st and st + n <= 2048 for st, n in segs)
    assert len(segs) == max(1, min(8, steps // 32))
    if len(segs) == 1:
        assert abs(segs[0][0] + steps / 2 - 1024) <= 1
    for key, fills in (("llama8b_q8", bench.FILLS_8B),):
        segs8 = bench.segments(key, steps, CONFIGS[key].context_length)
        assert sum(n for _, n in segs8) == steps and [p for p, _ in segs8] == list(fills)


def test_segments_reject_what_does_not_fit():
    with pytest.raises(ValueError):
        bench.segments("llama1b_q8", 0, 2304)
    with pytest.raises(ValueError):
        bench.segments("llama1b_q8", 2048, 2304)


def test_cpu_baseline_sample_stays_inside_the_context():
    """The CPU baseline decodes per_start steps from each start, then, with a time
    budget, further consecutive positions only up to the context's end."""
    from gpullama3_hip.model import synth_model
    from tests.harness import small
    shape = small("llama1b_q8", vocab=512, ctx=64)
    tensors = synth_model(shape, 3)
    wb = bench.weight_bytes(shape, tensor_specs(shape))
    _, n, _, nbytes = bench.cpu_decode_rate(shape, tensors, [0, 40], 4, 1)
    assert n == 8
    assert nbytes == 8 * wb + sum(bench.kv_bytes(shape, p, elem_bytes=4) for p in [0, 1, 2, 3, 40, 41, 42, 43])
    # a budget far beyond what the context allows: every position from the start to the end, once
    _, n, _, nbytes = bench.cpu_decode_rate(shape, tensors, [52], 4, 1, budget_s=1e4)
    assert n == 12
    assert nbytes == 12 * wb + sum(bench.kv_bytes(shape, p, elem_bytes=4) for p in range(52, 64))
