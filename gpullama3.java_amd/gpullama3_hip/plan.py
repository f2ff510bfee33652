"""Host-side mirror of the reference's TornadoVM execution plan, backed by the C ABI.

HipMasterPlan keeps the method names and meaning of
tornadovm/TornadoVMMasterPlan.java (initializeTornadoVMPlan :37-79,
tornadoVMForwardExecuteLayered :127-153, forceCopyInReadOnlyDataLayered
:180-195, freeTornadoExecutionPlan :200-202) and of
InferenceCore.forwardTornadoVM (inference/InferenceCore.java:582-589).  Errors
surface as the exception types the reference raises for the same conditions.
"""
import ctypes

import numpy as np

from . import _lib as L
from .model import FAMILY_MODEL_TYPE, ModelShape, gl3_config, kind_and_layer


def _raise(status):
    msg = L.load().gl3_last_error()
    msg = msg.decode() if msg else ""
    if status == L.ERR_INVALID_ARGUMENT:
        raise ValueError(msg)                     # IllegalArgumentException
    if status == L.ERR_UNSUPPORTED:
        raise NotImplementedError(msg)            # UnsupportedOperationException
    if status == L.ERR_OUT_OF_MEMORY:
        raise MemoryError(msg)                    # TornadoOutOfMemoryException
    raise L.Gl3Error(status, msg)                 # IllegalStateException


def _ok(status):
    if status != L.OK:
        _raise(status)


class HipMasterPlan:
    """One device plan: weights, fp16 KV cache and the per-token schedule."""

    def __init__(self, shape: ModelShape, flags=0):
        self.lib = L.load()
        self.shape = shape
        self.flags = flags
        cfg = gl3_config(shape, flags)
        h = ctypes.c_void_p()
        _ok(self.lib.gl3_create(ctypes.byref(cfg), ctypes.byref(h)))
        self.h = h
        self._logits = np.zeros(shape.vocab_size, dtype=np.float32)

    # -- TornadoVMMasterPlan.initializeTornadoVMPlan: create + weight copy-in
    @classmethod
    def initialize_plan(cls, shape: ModelShape, tensors, flags=0, rope_tables=None):
        """tensors: {gguf name: (TensorSpec, uint8 array)} (e.g. GGUFFile.tensors or model.synth_model)."""
        plan = cls(shape, flags)
        try:
            for name, (spec, data) in tensors.items():
                plan.upload(name, spec.ggml_type, data)
            if rope_tables is not None:
                plan.set_rope_tables(*rope_tables)
            plan.force_copy_in_read_only_data()
        except BaseException:
            plan.free_execution_plan()
            raise
        return plan

    # -- ModelLoader.loadModel + initializeTornadoVMPlan, done by the library from a path
    @classmethod
    def from_gguf(cls, path, context_length=-1, flags=0):
        """Plan built straight from a GGUF file (gl3_create_from_gguf): the library
        parses it, maps it read-only and uploads every tensor from the mapping."""
        cfg = gguf_config(path, context_length, flags)
        plan = cls.__new__(cls)
        plan.lib = L.load()
        plan.shape = shape_of_config(cfg)
        plan.flags = flags
        h = ctypes.c_void_p()
        _ok(plan.lib.gl3_create_from_gguf(str(path).encode(), context_length, flags, ctypes.byref(h)))
        plan.h = h
        plan._logits = np.zeros(plan.shape.vocab_size, dtype=np.float32)
        return plan

    def upload(self, name, ggml_type, data):
        kind, layer = kind_and_layer(name)
        arr = np.ascontiguousarray(data)
        _ok(self.lib.gl3_upload(self.h, kind, layer, ctypes.c_void_p(arr.ctypes.data), arr.nbytes, ggml_type))

    def set_rope_tables(self, cos_table, sin_table):
        c = np.ascontiguousarray(cos_table, dtype=np.float32)
        s = np.ascontiguousarray(sin_table, dtype=np.float32)
        _ok(self.lib.gl3_set_rope_tables(self.h, L.fptr(c), L.fptr(s), c.shape[0], c.shape[1]))

    # -- forceCopyInReadOnlyDataLayered
    def force_copy_in_read_only_data(self):
        _ok(self.lib.gl3_prepare(self.h))

    # -- InferenceCore.forwardTornadoVM + tornadoVMForwardExecuteLayered
    def forward_execute_layered(self, token, position):
        """Logits (fp32 [vocab]) of one decode step; the array is reused by the next call."""
        _ok(self.lib.gl3_forward(self.h, token, position, L.fptr(self._logits), None))
        return self._logits

    def forward(self, token, position, logits=True):
        """(logits copy or None, greedy token)."""
        am = np.zeros(1, dtype=np.int32)
        out = np.zeros(self.shape.vocab_size, dtype=np.float32) if logits else None
        _ok(self.lib.gl3_forward(self.h, token, position, L.fptr(out) if logits else None, L.iptr(am)))
        return out, int(am[0])

    def generate_greedy(self, token, position, n_steps):
        out = np.zeros(n_steps, dtype=np.int32)
        _ok(self.lib.gl3_generate_greedy(self.h, token, position, n_steps, L.iptr(out)))
        return out

    def prefill(self, tokens, position):
        """The prompt phase batched (gl3_prefill): K and V of tokens at position.., no logits."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        _ok(self.lib.gl3_prefill(self.h, L.iptr(t), t.size, position))

    def generate_from_prompt(self, prompt, position, n_gen):
        """The prompt forwarded on the device, then n_gen greedy tokens (gl3_generate_from_prompt)."""
        pr = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_gen, dtype=np.int32)
        _ok(self.lib.gl3_generate_from_prompt(self.h, L.iptr(pr), pr.size, position, n_gen, L.iptr(out)))
        return out

    def generate_sampled(self, prompt, position, n_gen, temperature, topp, coins):
        """The prompt forwarded on the device, then n_gen tokens sampled on the device
        (gl3_generate_sampled); coins[k] in [0, 1) is the draw of generated token k."""
        pr = np.ascontiguousarray(prompt, dtype=np.int32)
        c = np.ascontiguousarray(coins, dtype=np.float32)
        if c.size < n_gen:
            raise ValueError(f"{c.size} draws for {n_gen} tokens")
        out = np.zeros(n_gen, dtype=np.int32)
        _ok(self.lib.gl3_generate_sampled(self.h, L.iptr(pr), pr.size, position, n_gen, float(temperature),
                                          float(topp), L.fptr(c), L.iptr(out)))
        return out

    def timing(self):
        e = ctypes.c_double()
        k = ctypes.c_double()
        n = ctypes.c_int32()
        _ok(self.lib.gl3_get_timing(self.h, ctypes.byref(e), ctypes.byref(k), ctypes.byref(n)))
        return e.value, k.value, n.value

    def time_attention(self, layer, position, n_reps=20):
        """Average ms of the standalone attention kernel at `position` (gl3_time_attention;
        overwrites the cache row at `position`)."""
        ms = ctypes.c_double()
        _ok(self.lib.gl3_time_attention(self.h, layer, position, n_reps, ctypes.byref(ms)))
        return ms.value

    def phase_trace(self):
        """Per-phase durations (us) of the last persistent-kernel step (needs FLAG_PHASE_TRACE)."""
        out = np.zeros(16 + 10 * self.shape.n_layers, dtype=np.float64)
        n = ctypes.c_int32()
        _ok(self.lib.gl3_get_phase_trace(self.h, out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), out.size,
                                         ctypes.byref(n)))
        return out[:n.value]

    def phase_stamps(self):
        """Raw 100 MHz stamps [boundary][workgroup] of the last persistent-kernel step (needs FLAG_PHASE_TRACE)."""
        n_b = 4 + 10 * self.shape.n_layers
        out = np.zeros(n_b * 4096, dtype=np.uint64)
        ns = ctypes.c_int32()
        nw = ctypes.c_int32()
        _ok(self.lib.gl3_get_phase_stamps(self.h, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)), out.size,
                                          ctypes.byref(ns), ctypes.byref(nw)))
        return out[:ns.value * nw.value].reshape(ns.value, nw.value)

    def reset(self):
        _ok(self.lib.gl3_reset(self.h))

    def write_kv(self, layer, pos0, k, v):
        k = np.ascontiguousarray(k, dtype=np.uint16)
        v = np.ascontiguousarray(v, dtype=np.uint16)
        _ok(self.lib.gl3_write_kv(self.h, layer, pos0, k.shape[0], L.u16ptr(k), L.u16ptr(v)))

    def read_kv(self, layer, pos0, npos):
        k = np.zeros((npos, self.shape.kv_dim), dtype=np.uint16)
        v = np.zeros_like(k)
        _ok(self.lib.gl3_read_kv(self.h, layer, pos0, npos, L.u16ptr(k), L.u16ptr(v)))
        return k, v

    def fill_kv_normal(self, seed, npos):
        _ok(self.lib.gl3_fill_kv_normal(self.h, seed, npos))

    # -- freeTornadoExecutionPlan
    def free_execution_plan(self):
        if getattr(self, "h", None) is not None and self.h.value:
            self.lib.gl3_destroy(self.h)
            self.h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free_execution_plan()

    def __del__(self):
        try:
            self.free_execution_plan()
        except Exception:
            pass


def gguf_config(path, context_length=-1, flags=0):
    """gl3_config the library derives from a GGUF file (gl3_gguf_config; no GPU needed)."""
    cfg = L.Gl3Config()
    _ok(L.load().gl3_gguf_config(str(path).encode(), context_length, flags, ctypes.byref(cfg)))
    return cfg


def shape_of_config(cfg):
    """ModelShape of a gl3_config (the embedding type is not part of the config:
    it is taken to be the planner key, and tying is left unknown as False)."""
    family = {v: k for k, v in FAMILY_MODEL_TYPE.items()}.get(cfg.model_type, "llama")
    return ModelShape(family, cfg.dim, cfg.hidden_dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                      cfg.vocab_size, cfg.context_length, cfg.rms_norm_eps, cfg.rope_theta, cfg.weight_type,
                      cfg.weight_type, False, "")


def device_name():
    buf = ctypes.create_string_buffer(256)
    _ok(L.load().gl3_device_name(buf, 256))
    return buf.value.decode()


# ---- op-level entry points (one device kernel each, host buffers)

def op_dequant_q8_0(blocks, n):
    out = np.zeros(n, dtype=np.float32)
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    _ok(L.load().gl3_op_dequant_q8_0(ctypes.c_void_p(b.ctypes.data), n, L.fptr(out)))
    return out


def op_f16_to_f32(bits):
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.zeros(b.size, dtype=np.float32)
    _ok(L.load().gl3_op_f16_to_f32(L.u16ptr(b), b.size, L.fptr(out)))
    return out


def op_gemv(ggml_type, w, rows, cols, x, norm_w=None, eps=1e-5, mode=L.GEMV_STORE, y=None):
    wb = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out_rows = rows // 2 if mode == L.GEMV_SWIGLU else rows
    out = np.zeros(out_rows, dtype=np.float32) if y is None else np.array(y, dtype=np.float32, copy=True)
    nw = None if norm_w is None else np.ascontiguousarray(norm_w, dtype=np.float32)
    _ok(L.load().gl3_op_gemv(ggml_type, ctypes.c_void_p(wb.ctypes.data), rows, cols, L.fptr(x),
                             L.fptr(nw) if nw is not None else None, eps, mode, L.fptr(out)))
    return out


def op_sample(logits, temperature, topp, coins):
    """Device sampler on host logits, one token per draw (gl3_op_sample)."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    c = np.ascontiguousarray(coins, dtype=np.float32)
    out = np.zeros(c.size, dtype=np.int32)
    _ok(L.load().gl3_op_sample(L.fptr(x), x.size, float(temperature), float(topp), L.fptr(c), c.size, L.iptr(out)))
    return out


def op_attention(q, kcache, vcache, n_heads, n_kv_heads, head_dim, pos):
    """q: fp32 [n_heads*hd]; k/v cache: fp16 bits [pos+1][n_kv*hd]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(kcache, dtype=np.uint16)
    vc = np.ascontiguousarray(vcache, dtype=np.uint16)
    out = np.zeros(n_heads * head_dim, dtype=np.float32)
    _ok(L.load().gl3_op_attention(L.fptr(q), L.u16ptr(kc), L.u16ptr(vc), n_heads, n_kv_heads, head_dim, pos,
                                  L.fptr(out)))
    return out
