"""ctypes wrapper of the CPU oracle (liboracle.so, built from gl3_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
benchmark's CPU-baseline leg, always as the checker (never as the thing
measured on the GPU path, never as a fallback for it).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

FAMILY = {"llama": 0, "qwen3": 2, "phi3": 3}
KIND = {
    "token_embd.weight": 0, "output_norm.weight": 1, "output.weight": 2, "attn_norm.weight": 3,
    "attn_q.weight": 4, "attn_k.weight": 5, "attn_v.weight": 6, "attn_qkv.weight": 7, "attn_output.weight": 8,
    "attn_q_norm.weight": 9, "attn_k_norm.weight": 10, "ffn_norm.weight": 11, "ffn_gate.weight": 12,
    "ffn_up.weight": 13, "ffn_down.weight": 14,
}


class OrcConfig(ctypes.Structure):
    _fields_ = [("family", ctypes.c_int), ("dim", ctypes.c_int), ("hidden_dim", ctypes.c_int),
                ("n_layers", ctypes.c_int), ("n_heads", ctypes.c_int), ("n_kv_heads", ctypes.c_int),
                ("head_dim", ctypes.c_int), ("vocab_size", ctypes.c_int), ("context_length", ctypes.c_int),
                ("rms_norm_eps", ctypes.c_float), ("rope_theta", ctypes.c_double), ("weight_type", ctypes.c_int),
                ("embd_type", ctypes.c_int), ("output_type", ctypes.c_int), ("kv_fp16", ctypes.c_int),
                ("f16_exact", ctypes.c_int), ("n_threads", ctypes.c_int)]


class SampleInfo(ctypes.Structure):
    _fields_ = [("token_exact", ctypes.c_int), ("margin_exact", ctypes.c_double), ("quirk", ctypes.c_int),
                ("nucleus", ctypes.c_int), ("ref_shift", ctypes.c_double)]


_lib = None
_FP = ctypes.POINTER(ctypes.c_float)


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        lib = ctypes.CDLL(LIB_PATH)
        P, I, F, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
        sig = {
            "orc_create": (P, [ctypes.POINTER(OrcConfig)]),
            "orc_destroy": (None, [P]),
            "orc_set_tensor": (I, [P, I, I, P, I]),
            "orc_reset": (None, [P]),
            "orc_forward": (I, [P, I, I, _FP]),
            "orc_key_cache": (_FP, [P, I]),
            "orc_value_cache": (_FP, [P, I]),
            "orc_rope_real": (_FP, [P]),
            "orc_rope_imag": (_FP, [P]),
            "orc_f16_to_f32": (F, [ctypes.c_uint16]),
            "orc_f16_to_f32_daz": (F, [ctypes.c_uint16]),
            "orc_f32_to_f16": (ctypes.c_uint16, [F]),
            "orc_dequant_q8_0": (None, [P, SZ, _FP]),
            "orc_dot_q8_0": (F, [P, SZ, _FP, I]),
            "orc_dot_f16": (F, [P, SZ, _FP, I, I]),
            "orc_dot_scalar": (F, [_FP, _FP, I]),
            "orc_matmul": (None, [P, I, _FP, _FP, I, I, I]),
            "orc_rmsnorm": (None, [_FP, _FP, _FP, I, I, F]),
            "orc_rope_tables": (None, [I, I, ctypes.c_double, _FP, _FP]),
            "orc_softmax": (None, [_FP, I]),
            "orc_argmax": (I, [_FP, I]),
            "orc_attention_head": (None, [_FP, _FP, _FP, I, I, I, _FP, _FP]),
            "orc_sample": (I, [_FP, I, F, F, F, _FP, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(SampleInfo)]),
            "orc_set_simd": (None, [I]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def fp(a):
    return a.ctypes.data_as(_FP)


class OracleModel:
    """The reference's CPU forward on borrowed GGUF-encoded tensors."""

    def __init__(self, shape, tensors, kv_fp16=False, f16_exact=False, n_threads=0):
        self.lib = load()
        self.shape = shape
        out_type = tensors["output.weight"][0].ggml_type if "output.weight" in tensors else shape.embd_type
        c = OrcConfig(FAMILY[shape.family], shape.dim, shape.hidden_dim, shape.n_layers, shape.n_heads,
                      shape.n_kv_heads, shape.head_dim, shape.vocab_size, shape.context_length, shape.rms_norm_eps,
                      float(np.float32(shape.rope_theta)), shape.weight_type, shape.embd_type, out_type,
                      int(kv_fp16), int(f16_exact), n_threads)
        self.h = self.lib.orc_create(ctypes.byref(c))
        if not self.h:
            raise MemoryError("orc_create failed")
        self._keep = []
        for name, (spec, data) in tensors.items():
            arr = np.ascontiguousarray(data)
            self._keep.append(arr)
            if name.startswith("blk."):
                _, layer, rest = name.split(".", 2)
                kind, layer = KIND[rest], int(layer)
            else:
                kind, layer = KIND[name], 0
            if self.lib.orc_set_tensor(self.h, kind, layer, ctypes.c_void_p(arr.ctypes.data), spec.ggml_type):
                raise ValueError(name)
        self.logits = np.zeros(shape.vocab_size, dtype=np.float32)

    def forward(self, token, position):
        if self.lib.orc_forward(self.h, token, position, fp(self.logits)):
            raise ValueError(f"token {token} / position {position} out of range")
        return self.logits.copy()

    def reset(self):
        self.lib.orc_reset(self.h)

    def kv(self, layer):
        s = self.shape
        n = s.context_length * s.kv_dim
        k = np.ctypeslib.as_array(self.lib.orc_key_cache(self.h, layer), shape=(n,)).reshape(s.context_length, s.kv_dim)
        v = np.ctypeslib.as_array(self.lib.orc_value_cache(self.h, layer), shape=(n,)).reshape(s.context_length,
                                                                                               s.kv_dim)
        return k, v

    def rope_tables(self):
        s = self.shape
        n = s.context_length * (s.head_dim // 2)
        r = np.ctypeslib.as_array(self.lib.orc_rope_real(self.h), shape=(n,)).reshape(s.context_length, -1).copy()
        i = np.ctypeslib.as_array(self.lib.orc_rope_imag(self.h), shape=(n,)).reshape(s.context_length, -1).copy()
        return r, i

    def close(self):
        if self.h:
            self.lib.orc_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def matmul(w, ggml_type, x, rows, cols, f16_exact=False):
    lib = load()
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(rows, dtype=np.float32)
    wb = np.ascontiguousarray(w)
    lib.orc_matmul(ctypes.c_void_p(wb.ctypes.data), ggml_type, fp(x), fp(out), rows, cols, int(f16_exact))
    return out


def rmsnorm(x, w, eps, offset=0, size=None):
    lib = load()
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    size = x.size if size is None else size
    out = x.copy()
    lib.orc_rmsnorm(fp(out), fp(x), fp(w), offset, size, eps)
    return out


def rope_tables(ctx, head_size, theta):
    lib = load()
    cr = np.zeros(ctx * (head_size // 2), dtype=np.float32)
    ci = np.zeros_like(cr)
    lib.orc_rope_tables(ctx, head_size, float(theta), fp(cr), fp(ci))
    return cr.reshape(ctx, -1), ci.reshape(ctx, -1)


def attention_head(q, kcache, vcache, kv_stride, head_size, pos, offset=0):
    """One head over caches of row stride kv_stride, starting `offset` floats into each row."""
    lib = load()
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(kcache, dtype=np.float32)
    vc = np.ascontiguousarray(vcache, dtype=np.float32)
    assert kc.size >= pos * kv_stride + offset + head_size and vc.size == kc.size
    att = np.zeros(pos + 1, dtype=np.float32)
    out = np.zeros(head_size, dtype=np.float32)
    kp = ctypes.cast(kc.ctypes.data + 4 * offset, _FP)
    vp = ctypes.cast(vc.ctypes.data + 4 * offset, _FP)
    lib.orc_attention_head(fp(q), kp, vp, kv_stride, head_size, pos, fp(att), fp(out))
    return out


def softmax(x):
    lib = load()
    y = np.array(x, dtype=np.float32, copy=True)
    lib.orc_softmax(fp(y), y.size)
    return y


def argmax(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    return load().orc_argmax(fp(x), x.size)


def sample(logits, temperature, topp, coin):
    """The reference's Sampler on one logits vector for the draw `coin`:
    (token, exact token, exact margin, heap-order quirk, nucleus size); sample_info
    also returns the reference's float-sum shift at its decision."""
    lib = load()
    x = np.ascontiguousarray(logits, dtype=np.float32)
    n = x.size
    probs = np.zeros(n, dtype=np.float32)
    idx = np.zeros(n, dtype=np.int32)
    info = SampleInfo()
    tok = lib.orc_sample(fp(x), n, float(temperature), float(topp), float(coin), fp(probs),
                         idx.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), ctypes.byref(info))
    sample.last_shift = info.ref_shift
    return tok, info.token_exact, info.margin_exact, info.quirk, info.nucleus
