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


def lora_ranks(n_embd: int):
    """(w, a, v, g) low-rank sizes of an x070 block of width n_embd: the x070
    sizing rule max(32, round(c·n_embd^p / 32)·32) with (c, p) = (1.8, 0.5),
    (1.8, 0.5), (1.3, 0.5), (0.6, 0.8)."""
    def r(c, p):
        return max(32, int(round(c * n_embd ** p / 32)) * 32)
    return r(1.8, 0.5), r(1.8, 0.5), r(1.3, 0.5), r(0.6, 0.8)


def _f16(x):
    """Values representable in fp16 (as a parameter file in fp16 holds them), fp32."""
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def x070_dense_params(shape: "X070Shape", seed: int = 0, lora_dtype=np.float16):
    """Seeded non-projection parameters of an x070 model (the weights
    X070Generation reads with `gg`): layer norms, token-shift coefficients,
    low-rank branches (matrices in `lora_dtype`, fp16 as in an .rwkvq base),
    k_k / k_a / r_k, ln_x, the cmix coefficient and a fp16 embedding table.
    Vector parameters are fp16 values held in fp32."""
    rng = np.random.default_rng(seed)
    D, V = shape.n_embd, shape.vocab
    rw, ra, rv, rg = lora_ranks(D)
    n = lambda *s: rng.standard_normal(s, dtype=np.float32)
    p = {
        "emb.weight": (n(V, D) * 0.5).astype(np.float16),
        "ln0.weight": _f16(1 + 0.1 * n(D)), "ln0.bias": _f16(0.1 * n(D)),
        "ln_out.weight": _f16(1 + 0.1 * n(D)), "ln_out.bias": _f16(0.1 * n(D)),
    }
    mat = lambda o, i, s: (n(o, i) * np.float32(s)).astype(lora_dtype)
    for l in range(shape.n_layer):
        b = f"blocks.{l}."
        t = b + "tmix."
        for nm in ("ln1", "ln2"):
            p[b + nm + ".weight"] = _f16(1 + 0.1 * n(D))
            p[b + nm + ".bias"] = _f16(0.1 * n(D))
        for c in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"):
            p[t + c] = _f16(rng.uniform(0.0, 1.0, D))
        for nm, r in (("w", rw), ("a", ra), ("v", rv), ("g", rg)):
            p[t + nm + "_lora_A.weight"] = mat(r, D, 1.0 / np.sqrt(D))
            p[t + nm + "_lora_B.weight"] = mat(D, r, 0.5 / np.sqrt(r))
            if nm != "g":
                p[t + nm + "_lora_B.bias"] = _f16(0.5 * n(D))
        p[t + "k_k"] = _f16(1 + 0.1 * n(D))
        p[t + "k_a"] = _f16(1 + 0.1 * n(D))
        p[t + "r_k"] = _f16(0.1 * n(D))
        p[t + "ln_x.weight"] = _f16(1 + 0.1 * n(D))
        p[t + "ln_x.bias"] = _f16(0.1 * n(D))
        p[b + "cmix.x_k"] = _f16(rng.uniform(0.0, 1.0, D))
    return p


def x070_projections(shape: "X070Shape", nthreads: int = 8, share_layers: bool = False, seed0: int = 1000):
    """sb6 4-bit projections of an x070 model in the K3 layout: key → (qblk,
    qsqm, ddm, OUT, IN) for every decode GEMV (X070Shape.projections order),
    weights N(0, 0.02) seeded per matrix (seed0 + index).  `share_layers`
    reuses layer 0's packed bytes for the other layers (same traffic, less
    encoding time)."""
    from . import quant as Q

    out = {}
    for idx, (key, OUT, IN) in enumerate(shape.projections()):
        parts = key.split(".")
        if share_layers and parts[0] == "blocks" and parts[1] != "0":
            out[key] = out[".".join(["blocks", "0"] + parts[2:])]
            continue
        rng = np.random.default_rng(seed0 + idx)
        w = rng.standard_normal((OUT, IN), dtype=np.float32) * np.float32(0.02)
        disk = Q.encode_sb6(w, 4, nthreads)
        qblk, qsqm, ddm, _ = Q.rwkvq_sb6_to_k3(disk["codes_packed"], disk["gw_qsqm"], disk["gw_d"], disk["gw_dm"],
                                               None, None, (OUT, IN))
        out[key] = (qblk, qsqm, ddm, OUT, IN)
    return out
