"""Op-level parity of the device kernels against the oracle (through the C ABI)."""
import numpy as np
import pytest

import oracle.oracle as orc
from gpullama3_hip import _lib as L
from gpullama3_hip import plan as P
from gpullama3_hip.model import F16, Q8_0, TensorSpec, q8_0_blocks, synth_tensor

pytestmark = pytest.mark.gpu


def test_f16_to_f32_exhaustive(gpu):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = P.op_f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))  # subnormals kept
    assert np.all(np.isnan(got[~fin & np.isnan(ref)]))


def test_q8_0_dequant_bit_exact_exhaustive(gpu):
    scales = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    scales = scales[np.isfinite(scales.astype(np.float32))]
    qq = np.tile(np.arange(-128, 128, dtype=np.int8), scales.size)
    blocks = q8_0_blocks(qq, np.repeat(scales, 8))
    n = qq.size
    got = P.op_dequant_q8_0(blocks, n)
    ref = np.zeros(n, dtype=np.float32)
    orc.load().orc_dequant_q8_0(orc.ctypes.c_void_p(blocks.ctypes.data), n, orc.fp(ref))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


GEMV_COLS = [(Q8_0, c) for c in (1024, 2048, 3072, 4096, 8192, 14336)] + \
            [(F16, c) for c in (1024, 2048, 3072, 4096, 8192, 14336)] + \
            [(t, c) for t in (Q8_0, F16) for c in (1056, 2560, 9728)]  # widths of the any-length kernel


def make_w(t, rows, cols, seed):
    return synth_tensor(TensorSpec(f"g{seed}_{rows}_{cols}", t, rows, cols), seed)


def bound(w, t, rows, cols, x):
    import fp64_ref
    W = fp64_ref.dequant(TensorSpec("w", t, rows, cols), w).reshape(rows, cols)
    return np.abs(W) @ np.abs(x.astype(np.float64))


@pytest.mark.parametrize("t,cols", GEMV_COLS)
@pytest.mark.parametrize("mode", [L.GEMV_STORE, L.GEMV_RESIDUAL, L.GEMV_SWIGLU])
def test_gemv_vs_oracle(gpu, t, cols, mode):
    rows = 2 * 301 if mode == L.GEMV_SWIGLU else 333   # not a multiple of any row tile
    w = make_w(t, rows, cols, cols + mode)
    rng = np.random.default_rng(cols + 7 * mode)
    x = rng.standard_normal(cols).astype(np.float32)
    normw = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32) if mode != L.GEMV_RESIDUAL else None
    eps = 1e-5
    xin = orc.rmsnorm(x, normw, eps) if normw is not None else x
    full = orc.matmul(w, t, xin, rows, cols, f16_exact=True)
    b = bound(w, t, rows, cols, xin)
    tol = 2e-5 * b + 1e-7
    if mode == L.GEMV_STORE:
        got = P.op_gemv(t, w, rows, cols, x, normw, eps, mode)
        assert np.all(np.abs(got - full) <= tol)
    elif mode == L.GEMV_RESIDUAL:
        y0 = rng.standard_normal(rows).astype(np.float32)
        got = P.op_gemv(t, w, rows, cols, x, None, eps, mode, y=y0)
        assert np.all(np.abs(got - (y0 + full)) <= tol + 1e-6 * np.abs(y0))
    else:
        h = rows // 2
        g, u = full[:h].astype(np.float64), full[h:].astype(np.float64)
        ref = g / (1 + np.exp(-g)) * u
        got = P.op_gemv(t, w, rows, cols, x, normw, eps, mode)
        tg = tol[:h] * (np.abs(u) + 1) + tol[h:] * (np.abs(g) + 1)
        assert np.all(np.abs(got - ref) <= tg)


def test_gemv_rejects_unsupported_width(gpu):
    # past the any-length kernel's staging (15,872) and not a compiled tile width
    w = make_w(Q8_0, 4, 16384 + 1024, 1)
    with pytest.raises(NotImplementedError):
        P.op_gemv(Q8_0, w, 4, 16384 + 1024, np.zeros(16384 + 1024, np.float32))


def check_attention(hd, n_heads, n_kv, pos, seed):
    print(f"[case] attention hd={hd} heads={n_heads} kv_heads={n_kv} pos={pos}", flush=True)
    rng = np.random.Generator(np.random.SFC64(seed))
    kv_dim = n_kv * hd
    kc = rng.standard_normal((pos + 1, kv_dim), dtype=np.float32).astype(np.float16)
    vc = rng.standard_normal((pos + 1, kv_dim), dtype=np.float32).astype(np.float16)
    q = (rng.standard_normal(n_heads * hd) * 0.5).astype(np.float32)
    got = P.op_attention(q, kc.view(np.uint16), vc.view(np.uint16), n_heads, n_kv, hd, pos)
    G = n_heads // n_kv
    kf, vf = kc.astype(np.float32), vc.astype(np.float32)
    for h in range(n_heads):
        kvh = h // G
        ref = orc.attention_head(q[h * hd:(h + 1) * hd], kf, vf, kv_dim, hd, pos, offset=kvh * hd)
        assert np.max(np.abs(got[h * hd:(h + 1) * hd] - ref)) <= 2e-5 * np.abs(vc).max().astype(np.float32), h


# (head_dim, query heads, kv heads): GQA groups 4, 2, 1 (MHA), 4, 8 and 3 (Llama-3.2-3B)
@pytest.mark.parametrize("hd,n_heads,n_kv", [(64, 32, 8), (128, 16, 8), (96, 32, 32), (128, 32, 8), (64, 8, 8),
                                             (128, 32, 4), (64, 32, 4), (128, 24, 8)])
@pytest.mark.parametrize("pos", [0, 1, 63, 64, 200, 1500, 4095])
def test_attention_vs_oracle(gpu, hd, n_heads, n_kv, pos):
    check_attention(hd, n_heads, n_kv, pos, hd * 7919 + pos + 31 * n_kv)


# the Llama-3.1-8B attention shape (hd 128, GQA 4) and GQA 8 at the 16k and 32k KV fills:
# 16 and 32 splits of 1024 positions per kv head, merged by log-sum-exp
@pytest.mark.parametrize("hd,n_heads,n_kv", [(128, 32, 8), (128, 32, 4)])
@pytest.mark.parametrize("pos", [16383, 32767])
def test_attention_long_context_vs_oracle(gpu, hd, n_heads, n_kv, pos):
    check_attention(hd, n_heads, n_kv, pos, pos + n_kv)


def test_attention_one_position_is_exact(gpu):
    rng = np.random.default_rng(1)
    kc = rng.standard_normal((1, 512), dtype=np.float32).astype(np.float16)
    vc = rng.standard_normal((1, 512), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal(2048).astype(np.float32)
    got = P.op_attention(q, kc.view(np.uint16), vc.view(np.uint16), 32, 8, 64, 0)
    assert np.array_equal(got.reshape(32, 64), np.repeat(vc.astype(np.float32).reshape(8, 64), 4, axis=0))
