"""ctypes binding of libgpullama3_hip.so (the C ABI in include/gl3.h).

This is the Python counterpart of the Java FFM binding: every symbol of
include/gl3.h is declared here with its exact C signature.  Loading fails
loudly when the library has not been built; nothing here falls back to a CPU
implementation.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.normpath(os.path.join(_HERE, "..", "libgpullama3_hip.so"))

GL3_ABI_VERSION = 1

# gl3_status
OK, ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED, ERR_OUT_OF_MEMORY, ERR_DEVICE, ERR_STATE = range(6)

# gl3_model_type (model/ModelType.java order)
MODEL_LLAMA_3, MODEL_MISTRAL, MODEL_QWEN_3, MODEL_PHI_3, MODEL_QWEN_2, MODEL_DEEPSEEK_R1_DISTILL_QWEN = range(6)

# gl3_ggml_type
TYPE_F32, TYPE_F16, TYPE_Q8_0 = 0, 1, 8

# gl3_tensor_kind
(TOKEN_EMBD, OUTPUT_NORM, OUTPUT, ATTN_NORM, ATTN_Q, ATTN_K, ATTN_V, ATTN_QKV, ATTN_OUTPUT,
 ATTN_Q_NORM, ATTN_K_NORM, FFN_NORM, FFN_GATE, FFN_UP, FFN_DOWN) = range(15)

FLAG_PHASE_KERNELS = 1
FLAG_TIMING = 2
FLAG_PHASE_TRACE = 4
FLAG_STEPWISE_PROMPT = 8

GEMV_STORE, GEMV_RESIDUAL, GEMV_SWIGLU = 0, 1, 2


class Gl3Config(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("model_type", ctypes.c_int32),
        ("weight_type", ctypes.c_int32),
        ("dim", ctypes.c_int32),
        ("hidden_dim", ctypes.c_int32),
        ("n_layers", ctypes.c_int32),
        ("n_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("vocab_size", ctypes.c_int32),
        ("context_length", ctypes.c_int32),
        ("rms_norm_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float),
        ("flags", ctypes.c_uint32),
    ]


# symbol -> (restype, argtypes); the list every test checks against include/gl3.h
_P = ctypes.c_void_p
_I = ctypes.c_int
_SZ = ctypes.c_size_t
_FP = ctypes.POINTER(ctypes.c_float)
_IP = ctypes.POINTER(ctypes.c_int32)
_U16P = ctypes.POINTER(ctypes.c_uint16)
_DP = ctypes.POINTER(ctypes.c_double)

SIGNATURES = {
    "gl3_create": (_I, [ctypes.POINTER(Gl3Config), ctypes.POINTER(_P)]),
    "gl3_upload": (_I, [_P, _I, _I, _P, _SZ, _I]),
    "gl3_set_rope_tables": (_I, [_P, _FP, _FP, _I, _I]),
    "gl3_prepare": (_I, [_P]),
    "gl3_forward": (_I, [_P, ctypes.c_int32, ctypes.c_int32, _FP, _IP]),
    "gl3_generate_greedy": (_I, [_P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _IP]),
    "gl3_prefill": (_I, [_P, _IP, ctypes.c_int32, ctypes.c_int32]),
    "gl3_generate_from_prompt": (_I, [_P, _IP, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _IP]),
    "gl3_generate_sampled": (_I, [_P, _IP, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_float,
                                 ctypes.c_float, _FP, _IP]),
    "gl3_reset": (_I, [_P]),
    "gl3_write_kv": (_I, [_P, _I, _I, _I, _U16P, _U16P]),
    "gl3_read_kv": (_I, [_P, _I, _I, _I, _U16P, _U16P]),
    "gl3_fill_kv_normal": (_I, [_P, ctypes.c_uint64, _I]),
    "gl3_get_timing": (_I, [_P, _DP, _DP, _IP]),
    "gl3_get_phase_trace": (_I, [_P, _DP, ctypes.c_int32, _IP]),
    "gl3_get_phase_stamps": (_I, [_P, ctypes.POINTER(ctypes.c_uint64), ctypes.c_int64, _IP, _IP]),
    "gl3_time_attention": (_I, [_P, _I, ctypes.c_int32, ctypes.c_int32, _DP]),
    "gl3_gguf_config": (_I, [ctypes.c_char_p, ctypes.c_int32, ctypes.c_uint32, ctypes.POINTER(Gl3Config)]),
    "gl3_create_from_gguf": (_I, [ctypes.c_char_p, ctypes.c_int32, ctypes.c_uint32, ctypes.POINTER(_P)]),
    "gl3_destroy": (None, [_P]),
    "gl3_last_error": (ctypes.c_char_p, []),
    "gl3_device_name": (_I, [ctypes.c_char_p, _SZ]),
    "gl3_op_dequant_q8_0": (_I, [_P, _SZ, _FP]),
    "gl3_op_f16_to_f32": (_I, [_U16P, _SZ, _FP]),
    "gl3_op_gemv": (_I, [_I, _P, _I, _I, _FP, _FP, ctypes.c_float, _I, _FP]),
    "gl3_op_sample": (_I, [_FP, ctypes.c_int32, ctypes.c_float, ctypes.c_float, _FP, ctypes.c_int32, _IP]),
    "gl3_op_attention": (_I, [_FP, _U16P, _U16P, _I, _I, _I, _I, _FP]),
    "gl3_op_attention_noalloc": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _P, _P]),
}

_lib = None


class Gl3Error(RuntimeError):
    """Raised for a non-zero gl3_status; .status holds the code."""

    def __init__(self, status, message):
        super().__init__(f"gl3 status {status}: {message}")
        self.status = status


def load():
    """Load libgpullama3_hip.so once; raise if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() (HIP extension missing)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(status):
    if status != OK:
        msg = load().gl3_last_error()
        raise Gl3Error(status, msg.decode() if msg else "")
    return status


def fptr(a):
    return a.ctypes.data_as(_FP)


def iptr(a):
    return a.ctypes.data_as(_IP)


def u16ptr(a):
    return a.ctypes.data_as(_U16P)


def vptr(a):
    return ctypes.c_void_p(a.ctypes.data)
