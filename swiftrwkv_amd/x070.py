"""The x070 decode step on the HIP path: X070Backbone.step / stepEager
(Sources/RWKVGen/X070Generation.swift:437-500) for an .rwkvq base with the
step kernels on, over N independent rows (one token each).

Per layer and token, eight launches through the C ABI:
  rwkv_x070_shift_mix (ln1 + token shift + six lerps, tmixStep :214-239)
  rwkv_sb6_gemv_fused  (r / k / v projections, decodeRKV)
  rwkv_x070_lora_in    (inner `lin` of the four low-rank branches, :256-276)
  rwkv_x070_tmix_core  (outer `lin`s, w / a / vv / gate, kk, k, v, WKV step,
                        tail, :256-294)
  rwkv_sb6_gemv_ep     (o_proj + residual add, :294 / :493)
  rwkv_x070_shift_mix  (ln2 + token shift + lerp, cmixStep :303-308)
  rwkv_sb6_gemv_ep     (ffn key, relu², :308-309)
  rwkv_sb6_gemv_ep     (ffn value + residual add, :309 / :496)
plus rwkv_layer_norm for emb + ln0 (:489-490) and ln_out, and the head GEMV.
Activations are fp32; low-rank matrices keep their dtype (fp16: the `lin`
narrowing of :248-253).  There is no CPU fallback: a missing library raises.
"""
from __future__ import annotations

from typing import Dict, Optional, Tuple

import numpy as np
import torch

from . import _lib

HEAD = 64
LN_EPS = 1e-5
LNX_EPS = 64e-5
_COEF_ORDER = ("r", "k", "v", "w", "a", "g")   # rwkv_x070_shift_mix's coefficient order


class RWKVState:
    """RWKVState (X070Generation.swift:27-45) for N rows, on the device:
    wkv [L, N, H, 64, 64] fp32, tmix_prev / cmix_prev [L, N, D] fp32 and the
    in-step v_first [N, D] (written by layer 0 of every step)."""

    def __init__(self, n_layer: int, n_rows: int, n_embd: int, device):
        H = n_embd // HEAD
        z = lambda *s: torch.zeros(s, dtype=torch.float32, device=device)
        self.wkv = z(n_layer, n_rows, H, HEAD, HEAD)
        self.tmix_prev = z(n_layer, n_rows, n_embd)
        self.cmix_prev = z(n_layer, n_rows, n_embd)
        self.v_first = z(n_rows, n_embd)

    @property
    def n_rows(self) -> int:
        return self.wkv.shape[1]

    def clone(self) -> "RWKVState":
        c = RWKVState.__new__(RWKVState)
        c.wkv, c.tmix_prev, c.cmix_prev, c.v_first = (t.clone() for t in (self.wkv, self.tmix_prev, self.cmix_prev,
                                                                            self.v_first))
        return c

    def copy_(self, other: "RWKVState") -> "RWKVState":
        for a, b in zip((self.wkv, self.tmix_prev, self.cmix_prev, self.v_first),
                        (other.wkv, other.tmix_prev, other.cmix_prev, other.v_first)):
            a.copy_(b)
        return self


def _dt(t: torch.Tensor) -> int:
    if t.dtype == torch.float16:
        return _lib.F16
    if t.dtype == torch.float32:
        return _lib.F32
    raise TypeError(f"low-rank matrices must be fp16 or fp32, got {t.dtype}")


class X070Decoder:
    """Device-resident x070 model (sb6 projections in K3 layout + dense
    parameters) and its one-token step.

    dense: the `gg` parameters by name (numpy; see synthetic.x070_dense_params
    for the names); proj: key → (qblk, qsqm, ddm, OUT, IN) K3 buffers of every
    projection (X070Shape.projections names, sb6 4-bit)."""

    def __init__(self, n_layer: int, n_embd: int, ffn: int, vocab: int, dense: Dict[str, np.ndarray],
                 proj: Dict[str, Tuple], device, xbits: int = 0):
        self.L, self.D, self.F, self.V = n_layer, n_embd, ffn, vocab
        self.H = n_embd // HEAD
        self.xbits = xbits
        self.device = torch.empty(0, device=device).device   # concrete index (cuda → cuda:N)
        dev = self.device
        f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)
        keep = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        self.emb = keep(dense["emb.weight"])
        if self.emb.dtype not in (torch.float16, torch.float32):
            raise TypeError("emb.weight must be fp16 or fp32")
        self.ln0 = (f32(dense["ln0.weight"]), f32(dense["ln0.bias"]))
        self.ln_out = (f32(dense["ln_out.weight"]), f32(dense["ln_out.bias"]))
        self.layers = []
        ranks = None
        for l in range(n_layer):
            b, t = f"blocks.{l}.", f"blocks.{l}.tmix."
            A = [dense[t + nm + "_lora_A.weight"] for nm in "wavg"]
            r = tuple(int(a.shape[0]) for a in A)
            ranks = ranks or r
            if r != ranks:
                raise ValueError("low-rank sizes differ between layers")
            lay = {
                "ln1": (f32(dense[b + "ln1.weight"]), f32(dense[b + "ln1.bias"])),
                "ln2": (f32(dense[b + "ln2.weight"]), f32(dense[b + "ln2.bias"])),
                "coef6": f32(np.stack([dense[t + "x_" + c] for c in _COEF_ORDER])),
                "ck": f32(dense[b + "cmix.x_k"]),
                "wcat": keep(np.concatenate(A, 0)),
                "B": [keep(dense[t + nm + "_lora_B.weight"]) for nm in "wavg"],
                "bias": [f32(dense[t + nm + "_lora_B.bias"]) for nm in "wav"],
                "k_k": f32(dense[t + "k_k"]), "k_a": f32(dense[t + "k_a"]), "r_k": f32(dense[t + "r_k"]),
                "lnx": (f32(dense[t + "ln_x.weight"]), f32(dense[t + "ln_x.bias"])),
            }
            dts = {lay["wcat"].dtype} | {m.dtype for m in lay["B"]}
            if len(dts) != 1:
                raise TypeError("low-rank matrices of a layer must share one dtype")
            self.layers.append(lay)
        self.ranks = ranks
        self.proj = {}
        for l in range(n_layer):
            keys = [f"blocks.{l}.att.{m}.weight" for m in ("receptance", "key", "value")]
            self.proj[f"blocks.{l}.att.rkv"] = self._k3([proj[k] for k in keys])
            for k in (f"blocks.{l}.att.output.weight", f"blocks.{l}.ffn.key.weight", f"blocks.{l}.ffn.value.weight"):
                self.proj[k] = self._k3([proj[k]])
        self.proj["head.weight"] = self._k3([proj["head.weight"]])
        self._bufs: Optional[dict] = None

    def _k3(self, parts):
        dev = self.device
        return (torch.from_numpy(np.concatenate([p[0] for p in parts])).to(dev),
                torch.from_numpy(np.concatenate([p[1] for p in parts])).to(dev),
                torch.from_numpy(np.concatenate([p[2] for p in parts]).view(np.uint16)).to(dev),
                sum(p[3] for p in parts), parts[0][4])

    def new_state(self, n_rows: int) -> RWKVState:
        return RWKVState(self.L, n_rows, self.D, self.device)

    def _buffers(self, N: int) -> dict:
        if self._bufs is None or self._bufs["N"] != N:
            dev, D = self.device, self.D
            z = lambda *s: torch.empty(s, dtype=torch.float32, device=dev)
            self._bufs = {"N": N, "x": z(N, D), "xrkv": z(N, 3, D), "xmix": z(N, 4, D), "y_rkv": z(N, 3 * D),
                          "la": z(N, sum(self.ranks)), "tout": z(N, D), "xk": z(N, D), "hk": z(N, self.F),
                          "xo": z(N, D), "xl": z(D), "logits": z(N, self.V)}
        return self._bufs

    def launch(self, ids: torch.Tensor, state: RWKVState, stream: Optional[int] = None) -> torch.Tensor:
        """Enqueue one step of N = len(ids) rows on `stream` (default: torch's
        current stream); returns the logits buffer [N, vocab] (overwritten by
        the next launch).  Graph-capturable: no allocation once the buffers
        for N exist, no host synchronisation."""
        if ids.dtype != torch.int32 or ids.device != self.device or ids.dim() != 1:
            raise ValueError("ids must be a 1-D int32 tensor on the decoder's device")
        N = ids.numel()
        if state.n_rows != N:
            raise ValueError(f"state holds {state.n_rows} rows, ids {N}")
        s = torch.cuda.current_stream(self.device).cuda_stream if stream is None else stream
        bf = self._buffers(N)
        L, D = _lib.lib(), self.D
        p = lambda t: t.data_ptr()
        x = bf["x"]
        emb_dt = _lib.F16 if self.emb.dtype == torch.float16 else _lib.F32
        _lib.check(L.rwkv_layer_norm(p(self.emb), emb_dt, p(ids), self.V, p(self.ln0[0]), p(self.ln0[1]), p(x),
                                     N, D, LN_EPS, s))
        for l, lay in enumerate(self.layers):
            _lib.check(L.rwkv_x070_shift_mix(p(x), p(lay["ln1"][0]), p(lay["ln1"][1]), p(state.tmix_prev[l]),
                                             p(lay["coef6"]), 6, p(bf["xrkv"]), p(bf["xmix"]), N, D, LN_EPS, s))
            q = self.proj[f"blocks.{l}.att.rkv"]
            _lib.check(L.rwkv_sb6_gemv_fused(p(bf["xrkv"]), N, p(q[0]), p(q[1]), p(q[2]), p(bf["y_rkv"]), q[3], q[4],
                                             self.xbits, D, s))
            self._tmix_core(l, lay, state, bf, N, s)
            self._gemv(f"blocks.{l}.att.output.weight", bf["tout"], x, 1, N, s)
            _lib.check(L.rwkv_x070_shift_mix(p(x), p(lay["ln2"][0]), p(lay["ln2"][1]), p(state.cmix_prev[l]),
                                             p(lay["ck"]), 1, p(bf["xk"]), None, N, D, LN_EPS, s))
            self._gemv(f"blocks.{l}.ffn.key.weight", bf["xk"], bf["hk"], 2, N, s)
            self._gemv(f"blocks.{l}.ffn.value.weight", bf["hk"], x, 1, N, s)
        _lib.check(L.rwkv_layer_norm(p(x), _lib.F32, None, 0, p(self.ln_out[0]), p(self.ln_out[1]), p(bf["xo"]),
                                     N, D, LN_EPS, s))
        self._gemv("head.weight", bf["xo"], bf["logits"], 0, N, s)
        return bf["logits"]

    def launches_per_token(self, N: int = 1) -> int:
        return 8 * self.L + 3

    def _tmix_core(self, l, lay, state, bf, N, s):
        L, p = _lib.lib(), (lambda t: t.data_ptr())
        rw, ra, rv, rg = self.ranks
        wdt = _dt(lay["wcat"])
        _lib.check(L.rwkv_x070_lora_in(p(bf["xmix"]), p(lay["wcat"]), wdt, rw, ra, rv, rg, int(l > 0), p(bf["la"]),
                                       N, self.D, s))
        Bm = lay["B"]
        _lib.check(L.rwkv_x070_tmix_core(p(bf["y_rkv"]), p(bf["la"]), p(Bm[0]), p(Bm[1]), p(Bm[2]), p(Bm[3]), wdt,
                                         rw, ra, rv, rg, p(lay["bias"][0]), p(lay["bias"][1]), p(lay["bias"][2]),
                                         p(lay["k_k"]), p(lay["k_a"]), p(lay["r_k"]), p(lay["lnx"][0]),
                                         p(lay["lnx"][1]), p(state.v_first), int(l == 0), p(state.wkv[l]),
                                         p(bf["tout"]), N, self.H, LNX_EPS, s))

    def _gemv(self, key, x, y, ep, N, s):
        q = self.proj[key]
        _lib.check(_lib.lib().rwkv_sb6_gemv_ep(x.data_ptr(), N, q[0].data_ptr(), q[1].data_ptr(), q[2].data_ptr(),
                                               y.data_ptr(), q[3], q[4], self.xbits, ep, s))

    def step(self, ids, state: RWKVState) -> torch.Tensor:
        """X070Backbone.step (X070Generation.swift:437-474): token ids [N]
        (ints or a device int32 tensor) → logits [N, vocab] (a new tensor);
        `state` advances by one token per row."""
        if not isinstance(ids, torch.Tensor):
            ids = torch.tensor(np.asarray(ids, np.int32).reshape(-1), device=self.device)
        return self.launch(ids.to(device=self.device, dtype=torch.int32).reshape(-1), state).clone()

