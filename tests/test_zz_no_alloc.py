"""gl3_op_attention_noalloc (device buffers, scratch in a static device array,
no allocation) against gl3_op_attention (host buffers, allocating) on the same
inputs: bit-identical outputs on two calls in a row, the second smaller, and
the cache row at `pos` appended from the new k and v."""
import ctypes

import numpy as np
import pytest

from gpullama3_hip import _lib as L
from gpullama3_hip import plan as P

pytestmark = pytest.mark.gpu


class Hip:
    """The HIP runtime libgpullama3_hip.so already loaded (device buffers for the test's inputs)."""

    def __init__(self):
        with open("/proc/self/maps") as f:
            paths = sorted({ln.split()[-1] for ln in f if "libamdhip64.so" in ln})
        assert paths, "libamdhip64 is not loaded"
        self.lib = ctypes.CDLL(paths[0])
        self.bufs = []

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        assert self.lib.hipMalloc(ctypes.byref(p), ctypes.c_size_t(nbytes)) == 0
        self.bufs.append(p)
        return p

    def h2d(self, dst, arr):
        a = np.ascontiguousarray(arr)
        assert self.lib.hipMemcpy(dst, ctypes.c_void_p(a.ctypes.data), ctypes.c_size_t(a.nbytes), 1) == 0

    def d2h(self, src, arr):
        assert self.lib.hipDeviceSynchronize() == 0
        assert self.lib.hipMemcpy(ctypes.c_void_p(arr.ctypes.data), src, ctypes.c_size_t(arr.nbytes), 2) == 0

    def free(self):
        for p in self.bufs:
            self.lib.hipFree(p)
        self.bufs = []


def device_layout(kc, vc, n_kv, hd, ctxp):
    """Reference rows [npos][n_kv*hd] -> K [n_kv][ctxp][hd] and V [n_kv][ctxp/16][hd][16] (fp16 bits)."""
    npos = kc.shape[0]
    K = np.zeros((n_kv, ctxp, hd), dtype=np.uint16)
    K[:, :npos] = kc.reshape(npos, n_kv, hd).transpose(1, 0, 2)
    V = np.zeros((n_kv, ctxp, hd), dtype=np.uint16)
    V[:, :npos] = vc.reshape(npos, n_kv, hd).transpose(1, 0, 2)
    Vt = V.reshape(n_kv, ctxp // 16, 16, hd).transpose(0, 1, 3, 2).copy()
    return K, Vt


def noalloc(hip, q, kc, vc, n_heads, n_kv, hd, pos, ctxp):
    lib = L.load()
    fn = lib.gl3_op_attention_noalloc
    K, Vt = device_layout(kc[:pos], vc[:pos], n_kv, hd, ctxp)  # rows < pos; row pos comes from qkv
    qkv = np.concatenate([q, kc[pos].view(np.float16).astype(np.float32),
                          vc[pos].view(np.float16).astype(np.float32)]).astype(np.float32)
    dq, dk, dv = hip.alloc(qkv.nbytes), hip.alloc(K.nbytes), hip.alloc(Vt.nbytes)
    dout = hip.alloc(n_heads * hd * 4)
    hip.h2d(dq, qkv)
    hip.h2d(dk, K)
    hip.h2d(dv, Vt)
    rc = fn(dq, dk, dv, n_heads, n_kv, hd, ctxp, pos, dout, None)
    assert rc == L.OK, lib.gl3_last_error()
    out = np.zeros(n_heads * hd, dtype=np.float32)
    hip.d2h(dout, out)
    K2, Vt2 = np.zeros_like(K), np.zeros_like(Vt)
    hip.d2h(dk, K2)
    hip.d2h(dv, Vt2)
    Kr, Vtr = device_layout(kc[:pos + 1], vc[:pos + 1], n_kv, hd, ctxp)
    return out, np.array_equal(K2, Kr) and np.array_equal(Vt2, Vtr)


def test_noalloc_matches_op_attention_twice(gpu):
    hip = Hip()
    try:
        # the second call is smaller (fewer positions, heads and a shorter head)
        for hd, n_heads, n_kv, pos, ctxp in ((128, 32, 8, 3000, 3008), (64, 16, 4, 300, 320)):
            print(f"[case] noalloc hd={hd} heads={n_heads} kv={n_kv} pos={pos}", flush=True)
            rng = np.random.default_rng(pos)
            kc = rng.standard_normal((pos + 1, n_kv * hd), dtype=np.float32).astype(np.float16).view(np.uint16)
            vc = rng.standard_normal((pos + 1, n_kv * hd), dtype=np.float32).astype(np.float16).view(np.uint16)
            q = (rng.standard_normal(n_heads * hd) * 0.5).astype(np.float32)
            ref = P.op_attention(q, kc, vc, n_heads, n_kv, hd, pos)
            got, appended = noalloc(hip, q, kc, vc, n_heads, n_kv, hd, pos, ctxp)
            assert appended
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
            hip.free()
    finally:
        hip.free()


def test_noalloc_rejects_beyond_the_scratch(gpu):
    fn = L.load().gl3_op_attention_noalloc
    one = ctypes.c_void_p(16)  # never dereferenced: the call fails its checks first
    assert fn(one, one, one, 32, 8, 128, 100, 3, one, None) == L.ERR_INVALID_ARGUMENT  # ctxp not a multiple of 16
    assert fn(one, one, one, 128, 128, 128, 112, 3, one, None) == L.ERR_INVALID_ARGUMENT  # 128 kv heads
    assert fn(None, one, one, 32, 8, 128, 112, 3, one, None) == L.ERR_INVALID_ARGUMENT
