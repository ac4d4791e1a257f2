"""fp64 restatement of the x070 decode step around the hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by
the cpu_baseline leg of bench.py, always as the reference results are
compared with, never by the product package swiftrwkv_amd/.

Follows Sources/RWKVGen/X070Generation.swift for an .rwkvq base with the step
kernels on (the `fused` branch of tmixStep, :278-294), with fp32 activations:
  * stepEager (:484-500): emb row → ln0 → per layer x += tmix(ln1 x),
    x += cmix(ln2 x) → ln_out → head;
  * tmixStep (:201-296): token shift (:214-216), the six lerps (:225-239), the
    r/k/v projections, the low-rank branches through `lin` (:248-276), the
    w / kk / k / v formulas (:262-281), the WKV step (wkv7StepForward) and the
    tail (wkvTail), o_proj;
  * cmixStep (:299-310): token shift, one lerp, relu(key)², value;
  * layerNorm_ (:505-515), l2normLast (:502-504).
`lin` (:248-253): for a matrix whose dtype differs from the activations' (fp16
matrices, fp32 activations) the input is rounded to fp16, multiplied, and the
product rounded to fp16 and widened; equal dtypes give the plain product.

Everything is fp64 except those fp16 rounding points.  The WKV step and the
tail are the pinned oracle functions oracle.wkv7_fwd_f64 (T = 1) and
oracle.wkv_tail_f64; projections use matrices dequantised by oracle.sb6_dequant.

Layer 0 of the reference with an fp16 parameter file computes its tmix in
fp16 arithmetic (x is fp16 until the first residual add); this restatement,
like the HIP path, keeps fp32/fp64 activations from the embedding on.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import oracle as O

HEAD = 64


def f16r(x) -> np.ndarray:
    """Round to fp16 (round-to-nearest-even) and widen back."""
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def layer_norm(x, w, b, eps=1e-5):
    """layerNorm_ (X070Generation.swift:511-514): (x − mean)/sqrt(var + eps)·w + b."""
    x = np.asarray(x, np.float64)
    mean = x.mean(-1, keepdims=True)
    var = ((x - mean) ** 2).mean(-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * np.asarray(w, np.float64) + np.asarray(b, np.float64)


def lin(y, m):
    """`lin` (X070Generation.swift:248-253) with the .rwkvq narrowing."""
    y = np.asarray(y, np.float64)
    if m.dtype == np.float16:
        return f16r(f16r(y) @ m.astype(np.float64).T)
    return y @ np.asarray(m, np.float64).T


def l2norm_heads(x, H):
    """l2normLast (:502-504) per head of 64."""
    g = np.asarray(x, np.float64).reshape(x.shape[:-1] + (H, HEAD))
    return (g / np.sqrt((g * g).sum(-1, keepdims=True) + 1e-12)).reshape(x.shape)


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


def decay(ww):
    """The per-step decay from the w branch's output (RWKVBlock.swift:207-210,
    X070Generation.swift:274, X070Backbone.swift:1132): exp(-0.606531 · σ(ww))."""
    return np.exp(-0.606531 * sigmoid(ww))


@dataclass
class State:
    """RWKVState (X070Generation.swift:27-45) for N rows: wkv [L, N, H, 64, 64],
    tmix_prev / cmix_prev [L, N, D], v_first [N, D] (written by layer 0)."""
    wkv: np.ndarray
    tmix_prev: np.ndarray
    cmix_prev: np.ndarray
    v_first: np.ndarray

    @staticmethod
    def zeros(L, N, H):
        D = H * HEAD
        return State(np.zeros((L, N, H, HEAD, HEAD)), np.zeros((L, N, D)), np.zeros((L, N, D)), np.zeros((N, D)))

    def copy(self):
        return State(self.wkv.copy(), self.tmix_prev.copy(), self.cmix_prev.copy(), self.v_first.copy())


def dequant_projections(proj):
    """key → (qblk, qsqm, ddm, OUT, IN) sb6 4-bit K3 buffers → key → fp64 [OUT, IN]."""
    return {k: O.sb6_dequant(q[0], q[1], q[2], q[3], q[4], 0).astype(np.float64) for k, q in proj.items()}


def shift_mix(x, prev, coefs):
    """Token shift and lerps (tmixStep :214-239, cmixStep :303-308) on the
    layer-normed rows x: returns ([x + (prev − x)·c for c in coefs], new prev)."""
    x = np.asarray(x, np.float64)
    xx = np.asarray(prev, np.float64) - x
    return [x + xx * np.asarray(c, np.float64) for c in coefs], x.copy()


def lora_in(p, l, mw, ma, mv, mg):
    """Inner `lin` of the four low-rank branches (:256-276) with their
    functions: tanh(lin(xw, w1)), lin(xa, a1), lin(xv, v1) (None at layer 0),
    sigmoid(lin(xg, g1))."""
    t = f"blocks.{l}.tmix."
    return (np.tanh(lin(mw, p[t + "w_lora_A.weight"])), lin(ma, p[t + "a_lora_A.weight"]),
            None if l == 0 else lin(mv, p[t + "v_lora_A.weight"]), sigmoid(lin(mg, p[t + "g_lora_A.weight"])))


def core(p, l, r, k0, v, la, v_first, wkv, H):
    """The rest of tmixStep up to o_proj (:256-294) from the projections r, k0,
    v [N, D] and the low-rank inner outputs la = (lw, la, lv, lg): returns
    (tail·gate [N, D], new wkv, v_first)."""
    t = f"blocks.{l}.tmix."
    N, D = r.shape
    lw, la_, lv, lg = la
    gate = lin(lg, p[t + "g_lora_B.weight"])
    if l == 0:
        v_first = v.copy()
    else:
        vv = sigmoid(lin(lv, p[t + "v_lora_B.weight"]) + p[t + "v_lora_B.bias"])
        v = v + (v_first - v) * vv
    a = sigmoid(lin(la_, p[t + "a_lora_B.weight"]) + p[t + "a_lora_B.bias"])
    ww = lin(lw, p[t + "w_lora_B.weight"]) + p[t + "w_lora_B.bias"]
    w = decay(ww)
    kk = l2norm_heads(k0 * p[t + "k_k"], H)
    k = k0 * (1.0 + (a - 1.0) * p[t + "k_a"])
    sh = lambda z: np.asarray(z, np.float64).reshape(N, 1, H, HEAD)
    out, wkv = O.wkv7_fwd_f64(sh(r), sh(w), sh(k), sh(v), sh(-kk), sh(kk * a), wkv)
    tail = O.wkv_tail_f64(out.reshape(N, D), r, k, v, p[t + "r_k"], p[t + "ln_x.weight"], p[t + "ln_x.bias"],
                          gate, N, H, HEAD, 64e-5)
    return tail, wkv, v_first


def tmix(p, W, l, x, st: State, H):
    """tmixStep (:201-296) on the layer-normed rows x [N, D]; updates st."""
    t = f"blocks.{l}.tmix."
    m, st.tmix_prev[l] = shift_mix(x, st.tmix_prev[l], [p[t + "x_" + c] for c in "rwkvag"])
    m = dict(zip("rwkvag", m))
    a_ = f"blocks.{l}.att."
    r = m["r"] @ W[a_ + "receptance.weight"].T
    k0 = m["k"] @ W[a_ + "key.weight"].T
    v = m["v"] @ W[a_ + "value.weight"].T
    la = lora_in(p, l, m["w"], m["a"], m["v"], m["g"])
    tail, st.wkv[l], st.v_first = core(p, l, r, k0, v, la, st.v_first, st.wkv[l], H)
    return tail @ W[a_ + "output.weight"].T


def cmix(p, W, l, x, st: State):
    """cmixStep (:299-310) on the layer-normed rows x [N, D]; updates st."""
    (xk,), st.cmix_prev[l] = shift_mix(x, st.cmix_prev[l], [p[f"blocks.{l}.cmix.x_k"]])
    h = np.maximum(xk @ W[f"blocks.{l}.ffn.key.weight"].T, 0.0)
    return (h * h) @ W[f"blocks.{l}.ffn.value.weight"].T


def step(p, W, ids, st: State, n_layer, H):
    """stepEager (:484-500) for N rows: ids [N] → logits [N, vocab]; st updated."""
    x = layer_norm(p["emb.weight"].astype(np.float64)[np.asarray(ids)], p["ln0.weight"], p["ln0.bias"])
    for l in range(n_layer):
        b = f"blocks.{l}."
        x = x + tmix(p, W, l, layer_norm(x, p[b + "ln1.weight"], p[b + "ln1.bias"]), st, H)
        x = x + cmix(p, W, l, layer_norm(x, p[b + "ln2.weight"], p[b + "ln2.bias"]), st)
    return layer_norm(x, p["ln_out.weight"], p["ln_out.bias"]) @ W["head.weight"].T


def sequence(p, W, ids, n_layer, H):
    """The same model over a whole sequence of one row at once (the parallel
    formulation, RWKVBlock.swift rwkvTmixForward / cmix with the token shift
    as a shifted copy of the sequence and the WKV over all T steps in one
    call), from the zero state.  Returns logits [T, vocab]."""
    T = len(ids)
    D = H * HEAD
    x = layer_norm(p["emb.weight"].astype(np.float64)[np.asarray(ids)], p["ln0.weight"], p["ln0.bias"])
    v_first = None
    for l in range(n_layer):
        b = f"blocks.{l}."
        t = b + "tmix."
        xl = layer_norm(x, p[b + "ln1.weight"], p[b + "ln1.bias"])
        shifted = np.concatenate([np.zeros((1, D)), xl[:-1]], 0)
        xx = shifted - xl
        m = {c: xl + xx * p[t + "x_" + c].astype(np.float64) for c in "rwkvag"}
        a_ = b + "att."
        r = m["r"] @ W[a_ + "receptance.weight"].T
        k0 = m["k"] @ W[a_ + "key.weight"].T
        v = m["v"] @ W[a_ + "value.weight"].T
        gate = lin(sigmoid(lin(m["g"], p[t + "g_lora_A.weight"])), p[t + "g_lora_B.weight"])
        if l == 0:
            v_first = v.copy()
        else:
            vv = sigmoid(lin(lin(m["v"], p[t + "v_lora_A.weight"]), p[t + "v_lora_B.weight"]) + p[t + "v_lora_B.bias"])
            v = v + (v_first - v) * vv
        a = sigmoid(lin(lin(m["a"], p[t + "a_lora_A.weight"]), p[t + "a_lora_B.weight"]) + p[t + "a_lora_B.bias"])
        ww = lin(np.tanh(lin(m["w"], p[t + "w_lora_A.weight"])), p[t + "w_lora_B.weight"]) + p[t + "w_lora_B.bias"]
        w = decay(ww)
        kk = l2norm_heads(k0 * p[t + "k_k"], H)
        k = k0 * (1.0 + (a - 1.0) * p[t + "k_a"])
        sh = lambda z: np.asarray(z, np.float64).reshape(1, T, H, HEAD)
        out, _ = O.wkv7_fwd_f64(sh(r), sh(w), sh(k), sh(v), sh(-kk), sh(kk * a), None)
        tail = O.wkv_tail_f64(out.reshape(T, D), r, k, v, p[t + "r_k"], p[t + "ln_x.weight"], p[t + "ln_x.bias"],
                              gate, T, H, HEAD, 64e-5)
        x = x + tail @ W[a_ + "output.weight"].T
        xl = layer_norm(x, p[b + "ln2.weight"], p[b + "ln2.bias"])
        xx = np.concatenate([np.zeros((1, D)), xl[:-1]], 0) - xl
        xk = xl + xx * p[b + "cmix.x_k"].astype(np.float64)
        h = np.maximum(xk @ W[b + "ffn.key.weight"].T, 0.0)
        x = x + (h * h) @ W[b + "ffn.value.weight"].T
    return layer_norm(x, p["ln_out.weight"], p["ln_out.bias"]) @ W["head.weight"].T


def prefill(p, W, ids, n_layer, H, f16_base=False):
    """The parallel pass over one prompt from the zero state, as the
    reference's prefill runs it for an .rwkvq base (rwkvTmixForward /
    rwkvCmixForward, RWKVBlock.swift:163-307; bodyWithState + the head of
    prefillBatch, BatchGenerate.swift:37-53): token shift as a shifted copy
    of the sequence, one WKV-7 pass over all T steps, the low-rank branches
    as plain products (fp32 activations times the fp16 matrices' exact
    values: no `lin` narrowing on this path), projections through baseProj:
      * f16_base (the long pass of baseMatmul, X070Backbone.swift:337-356):
        y = fp16(fp16(x) · fp16(W)ᵀ), fp16(W) the fp16 dequant; cmix's
        relu(·)² rounded to fp16 (it is the next product's fp16 input);
      * else the fp32 GEMV (short pass): y = x·Wᵀ, relu² unrounded;
    the head always the GEMV (decode: true).  Returns (logits of the last
    token [vocab], State with the WKV states, and the shift states taken at
    the last token)."""
    T, D = len(ids), H * HEAD
    W16 = {}

    def proj(y, key):
        if not f16_base:
            return y @ W[key].T
        if key not in W16:
            W16[key] = f16r(W[key])
        return f16r(f16r(y) @ W16[key].T)

    wide = lambda y, m: np.asarray(y, np.float64) @ np.asarray(m, np.float64).T
    st = State.zeros(n_layer, 1, H)
    x = layer_norm(p["emb.weight"].astype(np.float64)[np.asarray(ids)], p["ln0.weight"], p["ln0.bias"])
    v_first = None
    for l in range(n_layer):
        b = f"blocks.{l}."
        t = b + "tmix."
        a_ = b + "att."
        xl = layer_norm(x, p[b + "ln1.weight"], p[b + "ln1.bias"])
        st.tmix_prev[l, 0] = xl[-1]
        xx = np.concatenate([np.zeros((1, D)), xl[:-1]], 0) - xl
        m = {c: xl + xx * p[t + "x_" + c].astype(np.float64) for c in "rwkvag"}
        r = proj(m["r"], a_ + "receptance.weight")
        k0 = proj(m["k"], a_ + "key.weight")
        v = proj(m["v"], a_ + "value.weight")
        gate = wide(sigmoid(wide(m["g"], p[t + "g_lora_A.weight"])), p[t + "g_lora_B.weight"])
        if l == 0:
            v_first = v.copy()
        else:
            vv = sigmoid(wide(wide(m["v"], p[t + "v_lora_A.weight"]), p[t + "v_lora_B.weight"]) + p[t + "v_lora_B.bias"])
            v = v + (v_first - v) * vv
        a = sigmoid(wide(wide(m["a"], p[t + "a_lora_A.weight"]), p[t + "a_lora_B.weight"]) + p[t + "a_lora_B.bias"])
        ww = wide(np.tanh(wide(m["w"], p[t + "w_lora_A.weight"])), p[t + "w_lora_B.weight"]) + p[t + "w_lora_B.bias"]
        w = decay(ww)
        kk = l2norm_heads(k0 * p[t + "k_k"], H)
        k = k0 * (1.0 + (a - 1.0) * p[t + "k_a"])
        sh = lambda z: np.asarray(z, np.float64).reshape(1, T, H, HEAD)
        out, st.wkv[l] = O.wkv7_fwd_f64(sh(r), sh(w), sh(k), sh(v), sh(-kk), sh(kk * a), None)
        tail = O.wkv_tail_f64(out.reshape(T, D), r, k, v, p[t + "r_k"], p[t + "ln_x.weight"], p[t + "ln_x.bias"],
                              gate, T, H, HEAD, 64e-5)
        x = x + proj(tail, a_ + "output.weight")
        xl = layer_norm(x, p[b + "ln2.weight"], p[b + "ln2.bias"])
        st.cmix_prev[l, 0] = xl[-1]
        xk = xl + (np.concatenate([np.zeros((1, D)), xl[:-1]], 0) - xl) * p[b + "cmix.x_k"].astype(np.float64)
        h = np.maximum(proj(xk, b + "ffn.key.weight"), 0.0)
        h = f16r(h * h) if f16_base else h * h
        x = x + proj(h, b + "ffn.value.weight")
    logits = layer_norm(x[-1:], p["ln_out.weight"], p["ln_out.bias"]) @ W["head.weight"].T
    return logits[0], st
