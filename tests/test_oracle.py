"""Pins the CPU oracle (oracle/gl3_oracle.c) before it is trusted as the checker.

Checks: exhaustive fp16 decode against numpy's IEEE conversion, exhaustive
Q8_0 dequantisation (every fp16 scale x every int8) against exact float64
products, dots and matmuls against float64 brute force, closed forms of
RMSNorm / RoPE / softmax / attention, lane-structure identity of the AVX2 and
portable code, the golden fixtures of tiny models of every family, and
sensitivity: a plausible mistake (wrong RoPE pairing, wrong theta, wrong eps,
dropped norm weight) makes the golden comparison fail.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle.oracle as orc
from gpullama3_hip.model import F16, F32, Q8_0, TensorSpec, q8_0_blocks, synth_model, synth_tensor
from golden.make_golden import SEED, TINY, sequence, weights_digest

GOLDEN_TOL = 1e-4  # max |oracle - fp64| relative to the logits std
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def lib():
    return orc.load()


def all_f16_bits():
    return np.arange(65536, dtype=np.uint32).astype(np.uint16)


def test_f16_decode_exhaustive(lib):
    bits = all_f16_bits()
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.orc_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


def test_f16_daz_decode(lib):
    bits = all_f16_bits()
    exp0 = (bits & 0x7C00) == 0
    fin = (bits & 0x7C00) != 0x7C00
    got = np.array([lib.orc_f16_to_f32_daz(int(b)) for b in bits], dtype=np.float32)
    ref = bits.view(np.float16).astype(np.float32)
    sel = fin & ~exp0
    assert np.array_equal(got[sel].view(np.uint32), ref[sel].view(np.uint32))
    # subnormals and zeros become signed zeros
    assert np.all(got[exp0] == 0.0)
    assert np.array_equal(np.signbit(got[exp0]), (bits[exp0] & 0x8000) != 0)


def test_f32_to_f16_rounding(lib):
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s for s in (1e-8, 1e-6, 1e-4, 1e-2, 1, 1e4)])
    xs = np.concatenate([xs, np.float32([0.0, -0.0, 65504, 65520, 70000, -1e-8, 5.96e-8, 2.98e-8])])
    got = np.array([lib.orc_f32_to_f16(float(x)) for x in xs], dtype=np.uint16)
    with np.errstate(over="ignore"):
        ref = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_q8_0_dequant_exhaustive(lib):
    """Every fp16 scale (incl. the ~30% subnormal scales of the Q8_0 configs) x every int8."""
    scales = all_f16_bits().view(np.float16)
    finite = np.isfinite(scales.astype(np.float32))
    scales = scales[finite]
    q = np.tile(np.arange(-128, 128, dtype=np.int8), 1)
    nb = scales.size * 8  # 256 quants per scale = 8 blocks
    qq = np.tile(q, scales.size)
    ss = np.repeat(scales, 8)
    blocks = q8_0_blocks(qq, ss)
    n = nb * 32
    out = np.zeros(n, dtype=np.float32)
    lib.orc_dequant_q8_0(ctypes.c_void_p(blocks.ctypes.data), n, orc.fp(out))
    exact = qq.astype(np.float64) * np.repeat(ss.astype(np.float64), 32)
    assert np.all(exact == exact.astype(np.float32).astype(np.float64)), "products exceed fp32 precision"
    assert np.array_equal(out.view(np.uint32), exact.astype(np.float32).view(np.uint32))


def rand_q8(rows, cols, seed):
    return synth_tensor(TensorSpec(f"w{seed}", Q8_0, rows, cols), seed)


def rand_f16(rows, cols, seed, std=0.02):
    return synth_tensor(TensorSpec(f"w{seed}", F16, rows, cols), seed, std=std)


def dq(data, t, rows, cols, daz=False):
    import fp64_ref
    return fp64_ref.dequant(TensorSpec("w", t, rows, cols), data, daz=daz).reshape(rows, cols)


@pytest.mark.parametrize("t", [Q8_0, F16])
def test_matmul_vs_fp64(lib, t):
    rows, cols = 37, 320
    w = rand_q8(rows, cols, 3) if t == Q8_0 else rand_f16(rows, cols, 3)
    x = np.random.default_rng(1).standard_normal(cols).astype(np.float32)
    got = orc.matmul(w, t, x, rows, cols)
    W = dq(w, t, rows, cols, daz=(t == F16))
    ref = W @ x.astype(np.float64)
    scale = np.abs(W) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(got - ref) <= 1e-6 * scale + 1e-30)


def test_matmul_one_hot_and_linearity(lib):
    rows, cols = 16, 256
    w = rand_q8(rows, cols, 5)
    W = dq(w, Q8_0, rows, cols)
    for j in (0, 31, 32, 200, 255):
        e = np.zeros(cols, dtype=np.float32)
        e[j] = 1.0
        assert np.array_equal(orc.matmul(w, Q8_0, e, rows, cols), W[:, j].astype(np.float32))
    x = np.random.default_rng(2).standard_normal(cols).astype(np.float32)
    assert np.array_equal(orc.matmul(w, Q8_0, 2 * x, rows, cols), 2 * orc.matmul(w, Q8_0, x, rows, cols))
    assert np.all(orc.matmul(w, Q8_0, np.zeros(cols, np.float32), rows, cols) == 0)


@pytest.mark.parametrize("t", [Q8_0, F16])
def test_simd_matches_portable_lane_structure(lib, t):
    rows, cols = 23, 1024
    w = rand_q8(rows, cols, 7) if t == Q8_0 else rand_f16(rows, cols, 7, std=1e-5)  # F16 with many subnormals
    x = np.random.default_rng(3).standard_normal(cols).astype(np.float32)
    lib.orc_set_simd(1)
    a = orc.matmul(w, t, x, rows, cols)
    lib.orc_set_simd(0)
    b = orc.matmul(w, t, x, rows, cols)
    lib.orc_set_simd(1)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q8_dot_unaligned_offset(lib):
    """The reference's alignment prologue (Q8_0FloatTensor.java:81-88) for offsets inside a block."""
    cols = 320
    w = rand_q8(1, cols, 11)
    W = dq(w, Q8_0, 1, cols)[0]
    x = np.random.default_rng(4).standard_normal(cols).astype(np.float32)
    for off in (1, 7, 31, 33):
        size = cols - off - 5
        got = lib.orc_dot_q8_0(ctypes.c_void_p(w.ctypes.data), off, orc.fp(x), size)
        ref = float(W[off:off + size] @ x[:size].astype(np.float64))
        assert abs(got - ref) <= 1e-5 * float(np.abs(W[off:off + size]) @ np.abs(x[:size]))


def test_f16_dot_daz_vs_exact(lib):
    cols = 64
    h = np.zeros(cols, dtype=np.float16)
    h[::2] = np.float16(3e-6)   # subnormal
    h[1::2] = np.float16(0.5)
    x = np.ones(cols, dtype=np.float32)
    daz = lib.orc_dot_f16(ctypes.c_void_p(h.ctypes.data), 0, orc.fp(x), cols, 0)
    exact = lib.orc_dot_f16(ctypes.c_void_p(h.ctypes.data), 0, orc.fp(x), cols, 1)
    assert daz == pytest.approx(16.0, abs=0)
    assert exact == pytest.approx(16.0 + 32 * float(np.float16(3e-6)), rel=1e-6)


def test_rmsnorm_closed_form(lib):
    c, eps, n = 0.37, 1e-5, 512
    x = np.full(n, c, dtype=np.float32)
    w = np.linspace(0.5, 1.5, n).astype(np.float32)
    got = orc.rmsnorm(x, w, eps)
    # sequential fp32 sum of 512 squares: relative error ~ n * 2^-24
    assert np.allclose(got, w * c / np.sqrt(c * c + eps), rtol=2e-5)
    xr = np.random.default_rng(5).standard_normal(n).astype(np.float32)
    ref = w * xr / np.sqrt(np.mean(xr.astype(np.float64) ** 2) + eps)
    assert np.allclose(orc.rmsnorm(xr, w, eps), ref, rtol=1e-5, atol=1e-7)


def test_rmsnorm_per_head_offset(lib):
    """Qwen3 per-head norm: weight index is index % size (InferenceCore.java:53)."""
    hd = 32
    x = np.random.default_rng(6).standard_normal(4 * hd).astype(np.float32)
    w = np.random.default_rng(7).standard_normal(hd).astype(np.float32)
    got = orc.rmsnorm(x, w, 1e-6, offset=2 * hd, size=hd)
    seg = x[2 * hd:3 * hd].astype(np.float64)
    assert np.allclose(got[2 * hd:3 * hd], w * seg / np.sqrt(np.mean(seg ** 2) + 1e-6), rtol=1e-5)
    assert np.array_equal(got[:2 * hd], x[:2 * hd]) and np.array_equal(got[3 * hd:], x[3 * hd:])


def test_rope_tables(lib):
    ctx, hs, theta = 64, 16, 500000.0
    cr, ci = orc.rope_tables(ctx, hs, theta)
    assert np.all(cr[0] == 1.0) and np.all(ci[0] == 0.0)
    assert np.allclose(cr ** 2 + ci ** 2, 1.0, atol=1e-6)
    i = np.arange(0, hs, 2)
    freq = (1.0 / theta ** (i / hs)).astype(np.float32)
    ang = (np.arange(ctx, dtype=np.float32)[:, None] * freq[None, :]).astype(np.float64)
    assert np.allclose(cr, np.cos(ang), atol=1e-6) and np.allclose(ci, np.sin(ang), atol=1e-6)


def test_softmax_and_argmax(lib):
    x = np.float32([1.0, 3.0, 2.0, 3.0, -1.0])
    p = orc.softmax(x)
    e = np.exp(x.astype(np.float64) - 3.0)
    assert np.allclose(p, e / e.sum(), rtol=1e-6)
    assert orc.argmax(x) == 1  # first maximum wins
    assert orc.argmax(np.float32([-5, -5, -7])) == 0


def test_attention_head_closed_forms(lib):
    hs, pos = 16, 9
    rng = np.random.default_rng(8)
    K = rng.standard_normal((pos + 1, hs)).astype(np.float32)
    V = rng.standard_normal((pos + 1, hs)).astype(np.float32)
    q = rng.standard_normal(hs).astype(np.float32)
    # pos = 0: out = V0 exactly
    assert np.array_equal(orc.attention_head(q, K, V, hs, hs, 0), V[0])
    # q = 0: mean of V
    assert np.allclose(orc.attention_head(np.zeros(hs, np.float32), K, V, hs, hs, pos), V.mean(0), rtol=1e-5,
                       atol=1e-6)
    # one dominant score returns that row
    K2 = K.copy()
    K2[4] = q * 100
    assert np.allclose(orc.attention_head(q, K2, V, hs, hs, pos), V[4], atol=1e-5)
    # float64 naive
    s = K.astype(np.float64) @ q / np.sqrt(hs)
    p = np.exp(s - s.max())
    ref = (p / p.sum()) @ V
    assert np.allclose(orc.attention_head(q, K, V, hs, hs, pos), ref, rtol=1e-5, atol=1e-6)


def golden(key):
    z = np.load(os.path.join(GOLDEN, f"tiny_{key}.npz"))
    return {k: z[k] for k in z.files}


def run_oracle(shape, tensors, toks, poss, **kw):
    m = orc.OracleModel(shape, tensors, **kw)
    out = np.stack([m.forward(int(t), int(p)) for t, p in zip(toks, poss)])
    m.close()
    return out


@pytest.mark.parametrize("key", sorted(TINY))
def test_oracle_matches_golden(key):
    g = golden(key)
    shape = TINY[key]
    tensors = synth_model(shape, int(g["seed"]), norm_init="random")
    assert weights_digest(tensors) == str(g["digest"]), "synthetic weight generator drifted"
    got = run_oracle(shape, tensors, g["tokens"], g["positions"])
    ref = g["logits"]
    tol = GOLDEN_TOL * ref.std()
    assert np.max(np.abs(got - ref)) <= tol
    assert np.array_equal(got.argmax(1), g["argmax"])


MUTATIONS = {
    "rope_theta": lambda s: s.with_(rope_theta=s.rope_theta * 0.1),
    "rms_eps": lambda s: s.with_(rms_norm_eps=s.rms_norm_eps * 1000 + 1e-2),
    "rope_pairing": lambda s: s.with_(family="qwen3" if s.family == "llama" else "llama"),
}


@pytest.mark.parametrize("mut", sorted(MUTATIONS))
@pytest.mark.parametrize("key", ["llama_q8", "phi3_f16"])
def test_golden_detects_planted_mistakes(key, mut):
    """A plausible mistake in the oracle's inputs must fail the golden comparison."""
    g = golden(key)
    shape = TINY[key]
    tensors = synth_model(shape, int(g["seed"]), norm_init="random")
    if mut == "rope_pairing" and shape.family == "phi3":
        pytest.skip("no model family has Phi3's fused tensors with interleaved RoPE")
    bad = MUTATIONS[mut](shape)
    if bad.family == "qwen3":
        # a Llama model run with NeoX pairing needs the per-head norms the qwen3 path reads: unit weights
        for l in range(shape.n_layers):
            for nm in ("attn_q_norm.weight", "attn_k_norm.weight"):
                sp = TensorSpec(f"blk.{l}.{nm}", F32, 1, shape.head_dim)
                tensors[sp.name] = (sp, np.ones(shape.head_dim, np.float32).view(np.uint8))
    got = run_oracle(bad, tensors, g["tokens"], g["positions"])
    assert np.max(np.abs(got - g["logits"])) > GOLDEN_TOL * g["logits"].std()


def test_dropped_norm_weight_is_detected():
    g = golden("llama_q8")
    shape = TINY["llama_q8"]
    tensors = synth_model(shape, int(g["seed"]), norm_init="random")
    sp = tensors["blk.1.ffn_norm.weight"][0]
    tensors["blk.1.ffn_norm.weight"] = (sp, np.ones(sp.cols, np.float32).view(np.uint8))
    got = run_oracle(shape, tensors, g["tokens"], g["positions"])
    assert np.max(np.abs(got - g["logits"])) > GOLDEN_TOL * g["logits"].std()


def test_kv_fp16_aid_close_to_reference():
    g = golden("qwen3_q8")
    shape = TINY["qwen3_q8"]
    tensors = synth_model(shape, int(g["seed"]), norm_init="random")
    got = run_oracle(shape, tensors, g["tokens"], g["positions"], kv_fp16=True)
    assert np.max(np.abs(got - g["logits"])) <= 2e-2 * g["logits"].std()


def test_sequence_helper_is_stable():
    toks, poss = sequence(TINY["llama_q8"], 4, 7)
    assert toks.dtype == np.int32 and list(poss) == [0, 1, 2, 3]
