"""C-ABI library checks that need no GPU: it loads, exports exactly the
functions include/gl3.h declares, and rejects invalid configurations with the
reference's error classes before touching the device."""
import ctypes
import os
import re

import numpy as np
import pytest

from gpullama3_hip import _lib as L
from gpullama3_hip.model import CONFIGS, gl3_config

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "gl3.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(gl3_[a-z0-9_]+)\s*\(", src)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(L.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = L.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = os.popen(f"nm -D --defined-only {L.LIB_PATH}").read()
    exported = set(re.findall(r"\bT (gl3_[a-z0-9_]+)", out))
    assert set(declared_functions()) <= exported


def test_config_struct_layout():
    assert ctypes.sizeof(L.Gl3Config) == 14 * 4
    src = open(HEADER).read()
    body = re.search(r"typedef struct gl3_config \{(.*?)\} gl3_config;", src, re.S).group(1)
    names = re.findall(r"\b(\w+);", body)
    assert names == [f[0] for f in L.Gl3Config._fields_]


def create(cfg):
    h = ctypes.c_void_p()
    rc = L.load().gl3_create(ctypes.byref(cfg), ctypes.byref(h))
    if rc == L.OK:
        L.load().gl3_destroy(h)
    return rc, L.load().gl3_last_error().decode()


@pytest.mark.parametrize("mutate,status", [
    (dict(model_type=L.MODEL_QWEN_2), L.ERR_UNSUPPORTED),
    (dict(model_type=L.MODEL_DEEPSEEK_R1_DISTILL_QWEN), L.ERR_UNSUPPORTED),
    (dict(model_type=99), L.ERR_INVALID_ARGUMENT),
    (dict(weight_type=L.TYPE_F32), L.ERR_UNSUPPORTED),
    (dict(weight_type=2), L.ERR_UNSUPPORTED),             # Q4_0: no GPU path in the reference either
    (dict(abi_version=7), L.ERR_INVALID_ARGUMENT),
    (dict(n_kv_heads=5), L.ERR_INVALID_ARGUMENT),
    (dict(head_dim=72), L.ERR_INVALID_ARGUMENT),           # head_dim * n_heads != dim for Llama
    (dict(context_length=0), L.ERR_INVALID_ARGUMENT),
    (dict(dim=2000, n_heads=20, n_kv_heads=4, head_dim=100), L.ERR_UNSUPPORTED),
    (dict(dim=1600, n_heads=25, n_kv_heads=5, head_dim=64), L.ERR_UNSUPPORTED),  # GQA group 5
])
def test_invalid_configs_rejected_without_device(mutate, status):
    cfg = gl3_config(CONFIGS["llama1b_q8"])
    for k, v in mutate.items():
        setattr(cfg, k, v)
    rc, msg = create(cfg)
    assert rc == status, msg
    assert msg


def test_null_arguments():
    lib = L.load()
    h = ctypes.c_void_p()
    assert lib.gl3_create(None, ctypes.byref(h)) == L.ERR_INVALID_ARGUMENT
    assert lib.gl3_forward(None, 0, 0, None, None) == L.ERR_INVALID_ARGUMENT
    assert lib.gl3_upload(None, 0, 0, None, 0, 1) == L.ERR_INVALID_ARGUMENT
    assert lib.gl3_op_gemv(L.TYPE_Q8_0, None, 4, 1024, None, None, 1e-5, 0, None) == L.ERR_INVALID_ARGUMENT
    lib.gl3_destroy(None)  # no-op
