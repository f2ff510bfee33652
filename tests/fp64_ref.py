"""Float64 brute-force forward pass used to pin the oracle on tiny models.

Independent of the oracle's code: weights are dequantised to float64 with
numpy, every operation is a whole-array numpy expression in float64, softmax
uses the max-shifted exponential.  It models the two places where the
reference's arithmetic is not plain real arithmetic on the stored values:
the FP16 vector dot flushes subnormal weights (FP16FloatTensor.java:91-98), and
the optional fp16 rounding of the KV cache (kv_fp16 test aid).
"""
import numpy as np

from gpullama3_hip.model import F16, F32, Q8_0, q8_0_unpack


def dequant(spec, data, daz=False):
    if spec.ggml_type == F32:
        return np.frombuffer(np.ascontiguousarray(data).tobytes(), dtype=np.float32).astype(np.float64)
    if spec.ggml_type == F16:
        h = np.frombuffer(np.ascontiguousarray(data).tobytes(), dtype=np.float16)
        v = h.astype(np.float64)
        if daz:
            sub = (h.view(np.uint16) & 0x7C00) == 0
            v = np.where(sub, 0.0, v)
        return v
    q, s = q8_0_unpack(data, spec.n)
    return q.astype(np.float64) * np.repeat(s.astype(np.float64), 32)


def rmsnorm(x, w, eps):
    return w * (x / np.sqrt(np.mean(x * x) + eps))


def rope_cs(pos, hs, theta):
    i = np.arange(0, hs, 2, dtype=np.float64)
    ang = pos * theta ** (-i / hs)
    return np.cos(ang), np.sin(ang)


class Fp64Model:
    def __init__(self, shape, tensors, kv_fp16=False):
        self.s = shape
        self.kv_fp16 = kv_fp16
        self.w = {}
        for name, (spec, data) in tensors.items():
            emb = name == "token_embd.weight"
            a = dequant(spec, data, daz=(spec.ggml_type == F16 and not emb))
            self.w[name] = a.reshape(spec.rows, spec.cols) if spec.rows > 1 else a
            if emb:  # the classifier reads token_embd through the (DAZ) vector dot when tied
                self.emb_exact = a.reshape(spec.rows, spec.cols)
                self.emb_daz = dequant(spec, data, daz=spec.ggml_type == F16).reshape(spec.rows, spec.cols)
        L, C, kv = shape.n_layers, shape.context_length, shape.kv_dim
        self.kc = np.zeros((L, C, kv))
        self.vc = np.zeros((L, C, kv))

    def _rot(self, vec, nheads, pos):
        s = self.s
        hs = s.head_dim
        c, si = rope_cs(pos, hs, np.float64(np.float32(s.rope_theta)))
        v = vec.reshape(nheads, hs).copy()
        if s.family == "llama":
            a, b = v[:, 0::2].copy(), v[:, 1::2].copy()
            v[:, 0::2], v[:, 1::2] = a * c - b * si, a * si + b * c
        else:
            h = hs // 2
            a, b = v[:, :h].copy(), v[:, h:].copy()
            v[:, :h], v[:, h:] = a * c - b * si, a * si + b * c
        return v.reshape(-1)

    def forward(self, token, pos):
        s, w = self.s, self.w
        hs, H = s.head_dim, s.hidden_dim
        x = self.emb_exact[token].copy()
        for l in range(s.n_layers):
            b = f"blk.{l}."
            xb = rmsnorm(x, w[b + "attn_norm.weight"], s.rms_norm_eps)
            if s.family == "phi3":
                qkv = w[b + "attn_qkv.weight"] @ xb
                q, k, v = qkv[:s.q_dim], qkv[s.q_dim:s.q_dim + s.kv_dim], qkv[s.q_dim + s.kv_dim:]
            else:
                q = w[b + "attn_q.weight"] @ xb
                k = w[b + "attn_k.weight"] @ xb
                v = w[b + "attn_v.weight"] @ xb
            if s.family == "qwen3":
                qn, kn = w[b + "attn_q_norm.weight"], w[b + "attn_k_norm.weight"]
                q = np.concatenate([rmsnorm(h, qn, s.rms_norm_eps) for h in q.reshape(s.n_heads, hs)])
                k = np.concatenate([rmsnorm(h, kn, s.rms_norm_eps) for h in k.reshape(s.n_kv_heads, hs)])
            q = self._rot(q, s.n_heads, pos)
            k = self._rot(k, s.n_kv_heads, pos)
            if self.kv_fp16:
                k = k.astype(np.float16).astype(np.float64)
                v = v.astype(np.float16).astype(np.float64)
            self.kc[l, pos], self.vc[l, pos] = k, v
            G = s.n_heads // s.n_kv_heads
            att = np.zeros(s.q_dim)
            for h in range(s.n_heads):
                kvh = h // G
                K = self.kc[l, :pos + 1, kvh * hs:(kvh + 1) * hs]
                V = self.vc[l, :pos + 1, kvh * hs:(kvh + 1) * hs]
                sc = K @ q[h * hs:(h + 1) * hs] / np.sqrt(hs)
                p = np.exp(sc - sc.max())
                p /= p.sum()
                att[h * hs:(h + 1) * hs] = p @ V
            x = x + w[b + "attn_output.weight"] @ att
            xb = rmsnorm(x, w[b + "ffn_norm.weight"], s.rms_norm_eps)
            if s.family == "phi3":
                gu = w[b + "ffn_up.weight"] @ xb
                g, u = gu[:H], gu[H:]
            else:
                g = w[b + "ffn_gate.weight"] @ xb
                u = w[b + "ffn_up.weight"] @ xb
            hb = g / (1.0 + np.exp(-g)) * u
            x = x + w[b + "ffn_down.weight"] @ hb
        x = rmsnorm(x, w["output_norm.weight"], s.rms_norm_eps)
        cls = w["output.weight"] if "output.weight" in w else self.emb_daz
        return cls @ x
