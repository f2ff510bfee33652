"""GGUF v3 writer and reader for synthetic models.

Follows the layout the reference parses (tensor/GGUF.java:43-92,217-311):
little-endian header {magic 'GGUF', version, tensor_count u64, kv_count u64},
key/value metadata, tensor infos {name, n_dims, dims (ne0 first), type, offset},
padding to general.alignment (32), then tensor data at aligned offsets.
The metadata satisfies the reference loaders: general.name selects the model
type (model/loader/ModelLoader.java:45-67), <arch>.* keys fill the
Configuration (LlamaModelLoader.java:47-62, Qwen3ModelLoader.java:48-73,
Phi3ModelLoader.java:45-60), and tokenizer.ggml.* arrays give the vocabulary.
"""
import mmap
import struct

import numpy as np

from .model import F16, F32, Q8_0, ModelShape, TensorSpec, tensor_specs, type_nbytes

MAGIC = 0x46554747
ALIGN = 32
# gguf_metadata_value_type
T_UINT8, T_INT8, T_UINT16, T_INT16, T_UINT32, T_INT32, T_FLOAT32, T_BOOL, T_STRING, T_ARRAY, T_UINT64, T_INT64, \
    T_FLOAT64 = range(13)

ARCH = {"llama": "llama", "qwen3": "qwen3", "phi3": "phi3"}
LLAMA_SPECIALS = {128000: "<|begin_of_text|>", 128001: "<|end_of_text|>", 128006: "<|start_header_id|>",
                  128007: "<|end_header_id|>", 128008: "<|eom_id|>", 128009: "<|eot_id|>"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key, vtype, value):
    out = _str(key) + struct.pack("<I", vtype)
    if vtype == T_STRING:
        out += _str(value)
    elif vtype == T_UINT32:
        out += struct.pack("<I", value)
    elif vtype == T_INT32:
        out += struct.pack("<i", value)
    elif vtype == T_FLOAT32:
        out += struct.pack("<f", value)
    elif vtype == T_ARRAY:
        etype, items = value
        out += struct.pack("<IQ", etype, len(items))
        if etype == T_STRING:
            out += b"".join(_str(x) for x in items)
        elif etype == T_INT32:
            out += np.asarray(items, dtype="<i4").tobytes()
        elif etype == T_FLOAT32:
            out += np.asarray(items, dtype="<f4").tobytes()
        else:
            raise ValueError(etype)
    else:
        raise ValueError(vtype)
    return out


def vocabulary(shape: ModelShape):
    toks = [f"t{i}" for i in range(shape.vocab_size)]
    if shape.family == "llama":
        base = 128000
        for i in range(base, shape.vocab_size):
            toks[i] = f"<|reserved_special_token_{i - base}|>"
        for i, t in LLAMA_SPECIALS.items():
            if i < shape.vocab_size:
                toks[i] = t
    return toks


def metadata(shape: ModelShape):
    a = ARCH[shape.family]
    kv = [("general.architecture", T_STRING, a), ("general.name", T_STRING, shape.name or a),
          ("general.alignment", T_UINT32, ALIGN),
          (f"{a}.embedding_length", T_UINT32, shape.dim), (f"{a}.feed_forward_length", T_UINT32, shape.hidden_dim),
          (f"{a}.block_count", T_UINT32, shape.n_layers), (f"{a}.attention.head_count", T_UINT32, shape.n_heads),
          (f"{a}.attention.head_count_kv", T_UINT32, shape.n_kv_heads),
          (f"{a}.context_length", T_UINT32, shape.context_length),
          (f"{a}.attention.layer_norm_rms_epsilon", T_FLOAT32, shape.rms_norm_eps),
          (f"{a}.rope.freq_base", T_FLOAT32, shape.rope_theta)]
    if shape.family == "qwen3":
        kv += [(f"{a}.attention.key_length", T_UINT32, shape.head_dim),
               (f"{a}.attention.value_length", T_UINT32, shape.head_dim)]
    if shape.family == "llama":
        kv += [(f"{a}.vocab_size", T_UINT32, shape.vocab_size)]
    toks = vocabulary(shape)
    kv += [("tokenizer.ggml.model", T_STRING, "gpt2" if shape.family != "phi3" else "llama"),
           ("tokenizer.ggml.tokens", T_ARRAY, (T_STRING, toks)),
           ("tokenizer.ggml.token_type", T_ARRAY, (T_INT32, [1] * len(toks)))]
    if shape.family != "phi3":
        kv += [("tokenizer.ggml.merges", T_ARRAY, (T_STRING, ["t 1"]))]
    else:
        kv += [("tokenizer.ggml.scores", T_ARRAY, (T_FLOAT32, [0.0] * len(toks)))]
    return kv


def write_gguf(path, shape: ModelShape, tensors):
    """tensors: {name: (TensorSpec, uint8 array)}; written in tensor_specs order."""
    specs = [sp for sp in tensor_specs(shape) if sp.name in tensors]
    kvs = metadata(shape)
    head = struct.pack("<IIQQ", MAGIC, 3, len(specs), len(kvs)) + b"".join(_kv(*k) for k in kvs)
    infos = b""
    off = 0
    offsets = []
    for sp in specs:
        dims = [sp.cols] if sp.rows == 1 else [sp.cols, sp.rows]
        infos += _str(sp.name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", sp.ggml_type, off)
        offsets.append(off)
        off += (sp.nbytes + ALIGN - 1) // ALIGN * ALIGN
    with open(path, "wb") as f:
        f.write(head + infos)
        pad = (-f.tell()) % ALIGN
        f.write(b"\0" * pad)
        base = f.tell()
        for sp, o in zip(specs, offsets):
            f.seek(base + o)
            f.write(np.ascontiguousarray(tensors[sp.name][1]).tobytes())
        end = base + off
        f.truncate(end)


class GGUFFile:
    """Read-only mmap of a GGUF file: .metadata, .tensors {name: (TensorSpec, uint8 view)}."""

    def __init__(self, path):
        self._f = open(path, "rb")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        buf = self._mm
        magic, version, n_t, n_kv = struct.unpack_from("<IIQQ", buf, 0)
        if magic != MAGIC:
            raise ValueError(f"unsupported header.magic {magic:#x}")
        if version not in (2, 3):
            raise ValueError(f"unsupported header.version {version}")
        p = 24
        self.metadata = {}

        def rd_str(p):
            (n,) = struct.unpack_from("<Q", buf, p)
            return bytes(buf[p + 8:p + 8 + n]).decode("utf-8"), p + 8 + n

        scalar = {T_UINT8: "<B", T_INT8: "<b", T_UINT16: "<H", T_INT16: "<h", T_UINT32: "<I", T_INT32: "<i",
                  T_FLOAT32: "<f", T_BOOL: "<?", T_UINT64: "<Q", T_INT64: "<q", T_FLOAT64: "<d"}

        def rd_val(t, p):
            if t == T_STRING:
                return rd_str(p)
            if t == T_ARRAY:
                et, n = struct.unpack_from("<IQ", buf, p)
                p += 12
                if et == T_STRING:
                    out = []
                    for _ in range(n):
                        s, p = rd_str(p)
                        out.append(s)
                    return out, p
                fmt = scalar[et]
                sz = struct.calcsize(fmt)
                return np.frombuffer(buf, dtype=np.dtype(fmt), count=n, offset=p).copy(), p + sz * n
            fmt = scalar[t]
            return struct.unpack_from(fmt, buf, p)[0], p + struct.calcsize(fmt)

        for _ in range(n_kv):
            k, p = rd_str(p)
            (t,) = struct.unpack_from("<I", buf, p)
            v, p = rd_val(t, p + 4)
            self.metadata[k] = v
        align = int(self.metadata.get("general.alignment", ALIGN))
        infos = []
        for _ in range(n_t):
            name, p = rd_str(p)
            (nd,) = struct.unpack_from("<I", buf, p)
            dims = struct.unpack_from(f"<{nd}Q", buf, p + 4)
            t, off = struct.unpack_from("<IQ", buf, p + 4 + 8 * nd)
            p += 4 + 8 * nd + 12
            infos.append((name, dims, t, off))
        data0 = p + (-p) % align
        self.tensors = {}
        for name, dims, t, off in infos:
            cols = dims[0]
            rows = int(np.prod(dims[1:])) if len(dims) > 1 else 1
            sp = TensorSpec(name, t, rows, cols)
            arr = np.frombuffer(buf, dtype=np.uint8, count=sp.nbytes, offset=data0 + off)
            self.tensors[name] = (sp, arr)

    def close(self):
        self.tensors = {}
        try:
            self._mm.close()
        except BufferError:
            pass
        self._f.close()
