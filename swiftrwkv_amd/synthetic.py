"""Seeded synthetic inputs and x070 shapes for tests and benchmarks.

Distributions follow the reference's own tests and the benchmark
configurations:
  * wkv_inputs_config0: r, k, v ~ N(0,1); w = exp(-exp(x)), x ~ U(-6,-1);
    kk = per-head L2-normalised N(0,1); a = -kk; b = kk·sigmoid(N(0,1)).
  * wkv_inputs_train: WKV7KernelParityTests.swift:15-30 / WKV7TrainKernelTests.swift:23-38
    (r, v, k ~ 0.5·N; a = -kk; b = kk·sigmoid(N); w = exp(-0.606531·sigmoid(N))).
  * wkv_inputs_seq: WKV7SequenceTests.swift:15-21 (0.3·N, w = exp(-|x|)).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

HEAD = 64


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _l2(x):
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + 1e-12)


def wkv_inputs_config0(B, T, H, seed=0):
    rng = np.random.default_rng(seed)
    n = lambda: rng.standard_normal((B, T, H, HEAD), dtype=np.float32)
    r, k, v = n(), n(), n()
    w = np.exp(-np.exp(rng.uniform(-6.0, -1.0, (B, T, H, HEAD)))).astype(np.float32)
    kk = _l2(n())
    a = (-kk).astype(np.float32)
    b = (kk * _sigmoid(n())).astype(np.float32)
    return [r, w, k, v, a, b]


def wkv_inputs_train(B, T, H, seed=0):
    rng = np.random.default_rng(seed)
    n = lambda s: (rng.standard_normal((B, T, H, HEAD), dtype=np.float32) * s).astype(np.float32)
    r, v, k = n(0.5), n(0.5), n(0.5)
    kk = _l2(k)
    a = (-kk).astype(np.float32)
    b = (kk * _sigmoid(n(1.0))).astype(np.float32)
    w = np.exp(-0.606531 * _sigmoid(n(1.0))).astype(np.float32)
    return [r, w, k, v, a, b]


def wkv_inputs_seq(B, T, H, seed=0):
    rng = np.random.default_rng(seed)
    x = [(rng.standard_normal((B, T, H, HEAD), dtype=np.float32) * 0.3).astype(np.float32) for _ in range(6)]
    x[1] = np.exp(-np.abs(x[1])).astype(np.float32)
    return x


def state(B, H, scale=0.1, seed=7):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((B, H, HEAD, HEAD), dtype=np.float32) * scale).astype(np.float32)


@dataclass(frozen=True)
class X070Shape:
    """x070 backbone sizes (BASELINE configurations)."""
    name: str
    n_layer: int
    n_embd: int
    ffn: int
    vocab: int = 65536

    @property
    def n_head(self) -> int:
        return self.n_embd // HEAD

    def projections(self):
        """(key, OUT, IN) of every decode GEMV of one token, in call order."""
        D, F = self.n_embd, self.ffn
        out = []
        for l in range(self.n_layer):
            for m in ("receptance", "key", "value", "output"):
                out.append((f"blocks.{l}.att.{m}.weight", D, D))
            out.append((f"blocks.{l}.ffn.key.weight", F, D))
            out.append((f"blocks.{l}.ffn.value.weight", D, F))
        out.append(("head.weight", self.vocab, D))
        return out


X070_0B1 = X070Shape("0.1B", 12, 768, 3072)
X070_0B4 = X070Shape("0.4B", 24, 1024, 4096)
X070_1B5 = X070Shape("1.5B", 24, 2048, 8192)
X070_7B = X070Shape("7B", 32, 4096, 14336)
