"""Model shapes, GGUF tensor naming and seeded synthetic weights.

The shapes mirror the reference's Configuration records
(model/llama/LlamaConfiguration.java, model/qwen3/Qwen3Configuration.java,
model/phi3/Phi3Configuration.java) and the tensor names are the ones its
loaders read (model/loader/LlamaModelLoader.java:77-98,
Qwen3ModelLoader.java:95-123, Phi3ModelLoader.java:102-122).  Tensors are held
in their GGUF encodings as uint8 arrays: F32, F16 (binary16) and Q8_0 (34-byte
blocks {fp16 scale, int8 q[32]}, tensor/GGMLType.java:13).
"""
from dataclasses import dataclass, field, replace
import hashlib

import numpy as np

from . import _lib as L

F32, F16, Q8_0 = L.TYPE_F32, L.TYPE_F16, L.TYPE_Q8_0

FAMILY_MODEL_TYPE = {"llama": L.MODEL_LLAMA_3, "qwen3": L.MODEL_QWEN_3, "phi3": L.MODEL_PHI_3}


@dataclass(frozen=True)
class ModelShape:
    family: str            # "llama" | "qwen3" | "phi3"
    dim: int
    hidden_dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    vocab_size: int
    context_length: int
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    weight_type: int = Q8_0    # all linear weights, incl. output.weight when untied
    embd_type: int = F16       # token_embd
    tied: bool = False         # no output.weight: the classifier is token_embd
    name: str = ""

    @property
    def q_dim(self):
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim

    def with_(self, **kw):
        return replace(self, **kw)


# The five workloads (Llama-3.2-1B F16 / Q8_0, Qwen3-0.6B Q8_0, Phi-3-mini F16, Llama-3.1-8B Q8_0).
CONFIGS = {
    "llama1b_f16": ModelShape("llama", 2048, 8192, 16, 32, 8, 64, 128256, 2048, 1e-5, 500000.0,
                              F16, F16, True, "Llama 3.2 1B (synthetic)"),
    "llama1b_q8": ModelShape("llama", 2048, 8192, 16, 32, 8, 64, 128256, 2048 + 256, 1e-5, 500000.0,
                             Q8_0, F16, False, "Llama 3.2 1B (synthetic)"),
    "qwen3_06b_q8": ModelShape("qwen3", 1024, 3072, 28, 16, 8, 128, 151936, 1024, 1e-6, 1000000.0,
                               Q8_0, F16, False, "Qwen3 0.6B (synthetic)"),
    "phi3_mini_f16": ModelShape("phi3", 3072, 8192, 32, 32, 32, 96, 32064, 4096 + 128, 1e-5, 10000.0,
                                F16, F16, False, "Phi-3-mini (synthetic)"),
    "llama8b_q8": ModelShape("llama", 4096, 14336, 32, 32, 8, 128, 128256, 32768 + 128, 1e-5, 500000.0,
                             Q8_0, F16, False, "Llama 3.1 8B (synthetic)"),
    # shapes on the per-phase schedule (no compiled persistent kernel): GQA group 3,
    # and row lengths outside the compiled GEMV tiles (dim 2560, hidden 9728)
    "llama3b_q8": ModelShape("llama", 3072, 8192, 28, 24, 8, 128, 128256, 4096, 1e-5, 500000.0,
                             Q8_0, F16, False, "Llama 3.2 3B (synthetic)"),
    "qwen3_4b_f16": ModelShape("qwen3", 2560, 9728, 36, 32, 8, 128, 151936, 4096, 1e-6, 1000000.0,
                               F16, F16, False, "Qwen3 4B (synthetic)"),
    # the other shapes of the reference's CI runs (build-and-run.yml)
    "phi3_mini_q8": ModelShape("phi3", 3072, 8192, 32, 32, 32, 96, 32064, 4096, 1e-5, 10000.0,
                               Q8_0, F16, False, "Phi-3-mini Q8_0 (synthetic)"),
    "mistral7b_f16": ModelShape("llama", 4096, 14336, 32, 32, 8, 128, 32768, 4096, 1e-5, 1000000.0,
                                F16, F16, False, "Mistral 7B v0.3 (synthetic)"),
}


def gl3_config(shape: ModelShape, flags=0):
    """gl3_config as the Java host fills it from the reference's Configuration."""
    return L.Gl3Config(L.GL3_ABI_VERSION, FAMILY_MODEL_TYPE[shape.family],
                       shape.embd_type if shape.tied else shape.weight_type,
                       shape.dim, shape.hidden_dim, shape.n_layers, shape.n_heads, shape.n_kv_heads,
                       shape.head_dim, shape.vocab_size, shape.context_length, shape.rms_norm_eps,
                       shape.rope_theta, flags)


KIND_OF = {
    "token_embd.weight": L.TOKEN_EMBD, "output_norm.weight": L.OUTPUT_NORM, "output.weight": L.OUTPUT,
    "attn_norm.weight": L.ATTN_NORM, "attn_q.weight": L.ATTN_Q, "attn_k.weight": L.ATTN_K,
    "attn_v.weight": L.ATTN_V, "attn_qkv.weight": L.ATTN_QKV, "attn_output.weight": L.ATTN_OUTPUT,
    "attn_q_norm.weight": L.ATTN_Q_NORM, "attn_k_norm.weight": L.ATTN_K_NORM, "ffn_norm.weight": L.FFN_NORM,
    "ffn_gate.weight": L.FFN_GATE, "ffn_up.weight": L.FFN_UP, "ffn_down.weight": L.FFN_DOWN,
}


def kind_and_layer(name):
    """GGUF tensor name -> (gl3_tensor_kind, layer)."""
    if name.startswith("blk."):
        _, layer, rest = name.split(".", 2)
        return KIND_OF[rest], int(layer)
    return KIND_OF[name], 0


@dataclass(frozen=True)
class TensorSpec:
    name: str
    ggml_type: int
    rows: int          # GGUF ne1 (1 for vectors)
    cols: int          # GGUF ne0

    @property
    def n(self):
        return self.rows * self.cols

    @property
    def nbytes(self):
        return type_nbytes(self.ggml_type, self.n)


def type_nbytes(t, n):
    return {F32: 4 * n, F16: 2 * n, Q8_0: n // 32 * 34}[t]


def tensor_specs(s: ModelShape):
    """All tensors of the model in GGUF order, with their types and shapes."""
    wt = s.weight_type
    specs = [TensorSpec("token_embd.weight", s.embd_type, s.vocab_size, s.dim),
             TensorSpec("output_norm.weight", F32, 1, s.dim)]
    if not s.tied:
        specs.append(TensorSpec("output.weight", wt, s.vocab_size, s.dim))
    for l in range(s.n_layers):
        b = f"blk.{l}."
        specs.append(TensorSpec(b + "attn_norm.weight", F32, 1, s.dim))
        if s.family == "phi3":
            specs.append(TensorSpec(b + "attn_qkv.weight", wt, s.q_dim + 2 * s.kv_dim, s.dim))
        else:
            specs.append(TensorSpec(b + "attn_q.weight", wt, s.q_dim, s.dim))
            specs.append(TensorSpec(b + "attn_k.weight", wt, s.kv_dim, s.dim))
            specs.append(TensorSpec(b + "attn_v.weight", wt, s.kv_dim, s.dim))
        if s.family == "qwen3":
            specs.append(TensorSpec(b + "attn_q_norm.weight", F32, 1, s.head_dim))
            specs.append(TensorSpec(b + "attn_k_norm.weight", F32, 1, s.head_dim))
        specs.append(TensorSpec(b + "attn_output.weight", wt, s.dim, s.q_dim))
        specs.append(TensorSpec(b + "ffn_norm.weight", F32, 1, s.dim))
        if s.family == "phi3":
            specs.append(TensorSpec(b + "ffn_up.weight", wt, 2 * s.hidden_dim, s.dim))
        else:
            specs.append(TensorSpec(b + "ffn_gate.weight", wt, s.hidden_dim, s.dim))
            specs.append(TensorSpec(b + "ffn_up.weight", wt, s.hidden_dim, s.dim))
        specs.append(TensorSpec(b + "ffn_down.weight", wt, s.dim, s.hidden_dim))
    return specs


def _rng(seed, name):
    h = hashlib.sha256(f"{seed}:{name}".encode()).digest()
    return np.random.Generator(np.random.PCG64(int.from_bytes(h[:8], "little")))


def q8_0_blocks(q, scales):
    """Pack int8 quants [n] and fp16 scales [n/32] into GGUF Q8_0 blocks (uint8 [n/32*34])."""
    nb = scales.size
    out = np.empty((nb, 34), dtype=np.uint8)
    out[:, :2] = scales.astype(np.float16).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = q.astype(np.int8).view(np.uint8).reshape(nb, 32)
    return out.reshape(-1)


def q8_0_unpack(blocks, n):
    """GGUF Q8_0 blocks -> (int8 quants [n], fp16 scales [n/32])."""
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, 34)[: n // 32]
    scales = b[:, :2].copy().view(np.float16).reshape(-1)
    q = b[:, 2:].copy().view(np.int8).reshape(-1)
    return q, scales


PAR_CHUNK = 1 << 22  # elements per independently seeded chunk of a large tensor


def _fill_chunk(spec, seed, out, i0, m, std):
    """Elements [i0, i0 + m) of a large linear weight, from the chunk's own SFC64
    stream (an order of magnitude faster than PCG64 here).  Q8_0 quants are raw
    random bytes as int8 with every -128 redrawn uniformly from [-127, 127], which
    is exactly U[-127, 127]."""
    h = hashlib.sha256(f"{seed}:{spec.name}#{i0 // PAR_CHUNK}".encode()).digest()
    bg = np.random.SFC64(int.from_bytes(h[:8], "little"))
    rng = np.random.Generator(bg)
    if spec.ggml_type == F16:
        out[i0:i0 + m] = rng.standard_normal(m, dtype=np.float32) * np.float32(std)
        return
    b0, nb = i0 // 32, m // 32
    sc = (np.abs(rng.standard_normal(nb, dtype=np.float32)) * np.float32(std / 127.0)).astype(np.float16)
    out[b0:b0 + nb, :2] = sc.view(np.uint8).reshape(nb, 2)
    q = bg.random_raw(m // 8).view(np.int8)
    bad = np.flatnonzero(q == -128)
    q[bad] = rng.integers(-127, 128, size=bad.size, dtype=np.int8)
    out[b0:b0 + nb, 2:] = q.view(np.uint8).reshape(nb, 32)


def _synth_large(spec, seed, std):
    """Tensors above PAR_CHUNK elements: chunks of PAR_CHUNK elements, each from its
    own seeded stream, generated on a thread pool (the generators release the GIL),
    so an 8B-parameter model takes seconds instead of minutes.  Same distributions
    as the single-stream path."""
    import concurrent.futures as cf
    import os
    n = spec.n
    out = np.empty(n, dtype=np.float16) if spec.ggml_type == F16 else np.empty((n // 32, 34), dtype=np.uint8)
    starts = range(0, n, PAR_CHUNK)
    workers = min(16, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(workers) as ex:
        list(ex.map(lambda i0: _fill_chunk(spec, seed, out, i0, min(PAR_CHUNK, n - i0), std), starts))
    return out.view(np.uint8).reshape(-1)


def synth_tensor(spec: TensorSpec, seed: int, norm_init="ones", std=0.02):
    """Seeded synthetic tensor in GGUF encoding.

    Linear weights: F16 ~ N(0, std); Q8_0 quants ~ U[-127, 127] with scales
    fp16(|N(0, std)| / 127).  Norm weights: 1.0 ("ones") or 1 + 0.1 N(0,1)
    ("random", used by the parity tests so a dropped norm weight is visible).
    Linear weights of more than PAR_CHUNK elements come from per-chunk streams
    (_synth_large).
    """
    n = spec.n
    if spec.ggml_type != F32 and n > PAR_CHUNK:
        return _synth_large(spec, seed, std)
    rng = _rng(seed, spec.name)
    if spec.ggml_type == F32:
        if norm_init == "ones":
            v = np.ones(n, dtype=np.float32)
        else:
            v = (1.0 + 0.1 * rng.standard_normal(n, dtype=np.float32)).astype(np.float32)
        return v.view(np.uint8)
    if spec.ggml_type == F16:
        out = np.empty(n, dtype=np.float16)
        step = 1 << 26
        for i in range(0, n, step):
            m = min(step, n - i)
            out[i:i + m] = rng.standard_normal(m, dtype=np.float32) * np.float32(std)
        return out.view(np.uint8)
    nb = n // 32
    out = np.empty((nb, 34), dtype=np.uint8)
    step = 1 << 21
    for i in range(0, nb, step):
        m = min(step, nb - i)
        sc = (np.abs(rng.standard_normal(m, dtype=np.float32)) * np.float32(std / 127.0)).astype(np.float16)
        out[i:i + m, :2] = sc.view(np.uint8).reshape(m, 2)
        out[i:i + m, 2:] = rng.integers(-127, 128, size=(m, 32), dtype=np.int8).view(np.uint8)
    return out.reshape(-1)


def synth_model(shape: ModelShape, seed=1234, norm_init="ones"):
    """{name: (TensorSpec, uint8 array)} for every tensor of the model."""
    return {sp.name: (sp, synth_tensor(sp, seed, norm_init)) for sp in tensor_specs(shape)}


def fp16_bits(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)
