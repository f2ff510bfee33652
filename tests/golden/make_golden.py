"""Writes the golden fixtures of tiny synthetic models (tests/golden/*.npz).

Each fixture holds the model shape, the weight seed and a sha256 of the
weights (to detect generator drift), the (token, position) sequence, the
float64 brute-force logits of every step (tests/fp64_ref.py) and the greedy
tokens.  The reference (Java + TornadoVM) cannot run here, so these vectors
come from an independent float64 restatement; the oracle is checked against
them and against closed forms in tests/test_oracle.py.

    python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "gpullama3.java_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

from gpullama3_hip.model import F16, Q8_0, ModelShape, synth_model  # noqa: E402
from fp64_ref import Fp64Model  # noqa: E402

TINY = {
    "llama_q8": ModelShape("llama", 64, 96, 2, 4, 2, 16, 101, 24, 1e-5, 500000.0, Q8_0, F16, False, "llama tiny"),
    "llama_f16_tied": ModelShape("llama", 64, 96, 2, 4, 2, 16, 101, 24, 1e-5, 500000.0, F16, F16, True, "llama tiny"),
    "qwen3_q8": ModelShape("qwen3", 64, 96, 2, 4, 2, 32, 113, 24, 1e-6, 1000000.0, Q8_0, F16, False, "qwen3 tiny"),
    "phi3_f16": ModelShape("phi3", 96, 64, 2, 4, 4, 24, 89, 24, 1e-5, 10000.0, F16, F16, False, "phi3 tiny"),
}
SEED = 20240601
STEPS = 12


def weights_digest(tensors):
    h = hashlib.sha256()
    for name in sorted(tensors):
        h.update(name.encode())
        h.update(np.ascontiguousarray(tensors[name][1]).tobytes())
    return h.hexdigest()


def sequence(shape, n, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, shape.vocab_size, size=n).astype(np.int32), np.arange(n, dtype=np.int32)


def main():
    for key, shape in TINY.items():
        tensors = synth_model(shape, SEED, norm_init="random")
        toks, poss = sequence(shape, STEPS, SEED + 1)
        m = Fp64Model(shape, tensors)
        logits = np.stack([m.forward(int(t), int(p)) for t, p in zip(toks, poss)])
        np.savez_compressed(os.path.join(HERE, f"tiny_{key}.npz"), logits=logits, tokens=toks, positions=poss,
                            argmax=logits.argmax(axis=1).astype(np.int32), seed=SEED,
                            digest=np.array(weights_digest(tensors)))
        print(key, logits.shape, float(logits.std()))


if __name__ == "__main__":
    main()
