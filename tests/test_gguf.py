"""GGUF reader of the library (gl3_gguf_config; no GPU): the configuration it
derives from a synthetic GGUF file equals the one the host builds from the same
shape, with the reference loaders' rules for context length, vocabulary, the
family and the planner key (model/loader/*ModelLoader.java, ModelLoader.java:45-67,
AbstractModelLoader.java:146-150), and malformed files fail with a status.
"""
import struct

import numpy as np
import pytest

from gpullama3_hip import _lib as L
from gpullama3_hip.gguf import GGUFFile, write_gguf
from gpullama3_hip.model import CONFIGS, gl3_config, synth_model
from gpullama3_hip.plan import gguf_config

FIELDS = ["abi_version", "model_type", "weight_type", "dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads",
          "head_dim", "vocab_size", "context_length", "rms_norm_eps", "rope_theta", "flags"]

# small shapes of the five families (GQA, Qwen3's q width != dim, Phi-3's MHA and head_dim 32)
TINY = {
    "llama1b_q8": CONFIGS["llama1b_q8"].with_(dim=128, hidden_dim=256, n_layers=2, n_heads=4, n_kv_heads=2,
                                              head_dim=32, vocab_size=300, context_length=64),
    "llama1b_f16": CONFIGS["llama1b_f16"].with_(dim=128, hidden_dim=256, n_layers=2, n_heads=4, n_kv_heads=2,
                                                head_dim=32, vocab_size=300, context_length=64, tied=True),
    "qwen3_06b_q8": CONFIGS["qwen3_06b_q8"].with_(dim=128, hidden_dim=192, n_layers=2, n_heads=4, n_kv_heads=2,
                                                  head_dim=64, vocab_size=320, context_length=96),
    "phi3_mini_f16": CONFIGS["phi3_mini_f16"].with_(dim=96, hidden_dim=128, n_layers=2, n_heads=3, n_kv_heads=3,
                                                    head_dim=32, vocab_size=256, context_length=64),
    "llama8b_q8": CONFIGS["llama8b_q8"].with_(dim=256, hidden_dim=512, n_layers=1, n_heads=8, n_kv_heads=2,
                                              head_dim=32, vocab_size=300, context_length=128),
}


def write(tmp_path, shape, name="m.gguf"):
    path = tmp_path / name
    write_gguf(path, shape, synth_model(shape, 5))
    return path


def as_dict(cfg):
    return {f: getattr(cfg, f) for f in FIELDS}


@pytest.mark.parametrize("key", sorted(TINY))
def test_config_matches_host(tmp_path, key):
    shape = TINY[key]
    path = write(tmp_path, shape)
    ctx = shape.context_length if shape.family == "phi3" else -1  # Phi-3 needs the requested length
    got = as_dict(gguf_config(path, ctx, L.FLAG_TIMING))
    want = as_dict(gl3_config(shape, L.FLAG_TIMING))
    assert got == want
    # the Python reader sees the same tensors the C reader uploads
    g = GGUFFile(path)
    assert set(g.tensors) == {n for n in synth_model(shape, 5)}
    g.close()


def test_context_length_rules(tmp_path):
    llama = TINY["llama1b_q8"]
    p = write(tmp_path, llama, "l.gguf")
    assert gguf_config(p, -1).context_length == llama.context_length   # the model's own
    assert gguf_config(p, 40).context_length == 40                     # withContextLength(40)
    assert gguf_config(p, 1000).context_length == 1000                 # Llama takes a longer one as given
    qwen = TINY["qwen3_06b_q8"]
    p = write(tmp_path, qwen, "q.gguf")
    assert gguf_config(p, 1000).context_length == qwen.context_length  # min(requested, model)
    assert gguf_config(p, 50).context_length == 50
    mistral = llama.with_(name="Mistral 7B (synthetic)")
    p = write(tmp_path, mistral, "m.gguf")
    c = gguf_config(p, 1000)
    assert c.model_type == L.MODEL_MISTRAL and c.context_length == mistral.context_length
    phi = TINY["phi3_mini_f16"]
    p = write(tmp_path, phi, "p.gguf")
    assert gguf_config(p, 200).context_length == 200                   # used as given
    with pytest.raises(ValueError):
        gguf_config(p, -1)


def test_family_detection_and_rejections(tmp_path):
    base = TINY["llama1b_q8"]
    for name, mt in (("Meta Llama 3.2", L.MODEL_LLAMA_3), ("mistral-7b", L.MODEL_MISTRAL)):
        assert gguf_config(write(tmp_path, base.with_(name=name), "a.gguf"), -1).model_type == mt
    for name in ("Qwen2.5 0.5B", "DeepSeek R1 Distill Qwen 1.5B", "gpt-something"):
        with pytest.raises(NotImplementedError):
            gguf_config(write(tmp_path, base.with_(name=name), "b.gguf"), -1)


def test_untied_output_type_is_the_planner_key(tmp_path):
    q8 = TINY["llama1b_q8"]          # F16 embeddings, Q8_0 output.weight
    assert gguf_config(write(tmp_path, q8, "a.gguf"), -1).weight_type == L.TYPE_Q8_0
    tied = TINY["llama1b_f16"]       # no output.weight: the embedding's type
    assert gguf_config(write(tmp_path, tied, "b.gguf"), -1).weight_type == L.TYPE_F16


def test_malformed_files(tmp_path):
    good = write(tmp_path, TINY["llama1b_q8"])
    data = good.read_bytes()
    bad_magic = tmp_path / "magic.gguf"
    bad_magic.write_bytes(b"GGUX" + data[4:])
    with pytest.raises(ValueError, match="magic"):
        gguf_config(bad_magic, -1)
    v1 = tmp_path / "v1.gguf"
    v1.write_bytes(data[:4] + struct.pack("<I", 1) + data[8:])
    with pytest.raises(NotImplementedError, match="version"):
        gguf_config(v1, -1)
    trunc = tmp_path / "trunc.gguf"
    trunc.write_bytes(data[:200])
    with pytest.raises(ValueError):
        gguf_config(trunc, -1)
    short = tmp_path / "short.gguf"          # header intact, tensor data cut off
    short.write_bytes(data[:len(data) - 4096])
    with pytest.raises(ValueError, match="past the end"):
        gguf_config(short, -1)
    with pytest.raises(ValueError, match="cannot open"):
        gguf_config(tmp_path / "missing.gguf", -1)


def test_fuzzed_headers_never_crash(tmp_path):
    """Random byte flips in the header and metadata either parse or fail with a status."""
    data = bytearray(write(tmp_path, TINY["qwen3_06b_q8"]).read_bytes())
    rng = np.random.default_rng(0)
    head = 4096
    for i in range(60):
        d = bytearray(data)
        for _ in range(4):
            d[int(rng.integers(8, head))] = int(rng.integers(0, 256))
        p = tmp_path / f"f{i}.gguf"
        p.write_bytes(bytes(d))
        try:
            gguf_config(p, -1)
        except (ValueError, NotImplementedError, L.Gl3Error, MemoryError):
            pass
