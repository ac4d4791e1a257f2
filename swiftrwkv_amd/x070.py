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
At batch 1 (4-bit sb6 r/k/v, fp16 low-rank matrices) the r/k/v GEMV and
lora_in are one launch, rwkv_x070_rkv_lora (seven per layer); with 4-bit
ffn key / value too, the r/k/v + low-rank and the ffn key launches form
their input rows themselves (rwkv_x070_rkv_lora_ln, rwkv_x070_ffn_key_ln;
the tmix core and rwkv_x070_ffn_value store the next token-shift rows):
five per layer, bitwise the same step.
Activations are fp32; low-rank matrices keep their dtype (fp16: the `lin`
narrowing of :248-253).  There is no CPU fallback: a missing library raises.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

from . import _lib
from . import quant as Q

HEAD = 64
LN_EPS = 1e-5
LNX_EPS = 64e-5
_COEF_ORDER = ("r", "k", "v", "w", "a", "g")   # rwkv_x070_shift_mix's coefficient order
# The parallel pass's low-rank branches take rwkv_x070_seq_lora's fp32 kernel
# (two launches, activations fused) up to this many rows × width: measured per
# layer, 0.1B width × 128 rows 16 µs (its K-split tiles) against 138 µs for the
# library GEMM, 1024 × 1024 60 against 66 µs.  Above it, passes with fp16 matrices take its
# two-part fp16 kernel (rwkv_x070_seq_lora_split); fp32 matrices the
# library's fp32 GEMM (4096 × 8192: 0.96 ms against 2.5 for the fp32 kernel).
SEQ_LORA_MAX_MD = 1 << 21


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

    def gather(self, rows) -> "RWKVState":
        """RWKVBatchState.gather: a new state of the listed rows, in that order
        (BatchGenerate.swift:105-108 drops the rows that stopped)."""
        idx = torch.as_tensor(list(rows), dtype=torch.long, device=self.wkv.device)
        c = RWKVState.__new__(RWKVState)
        c.wkv, c.tmix_prev, c.cmix_prev = (t.index_select(1, idx) for t in (self.wkv, self.tmix_prev, self.cmix_prev))
        c.v_first = self.v_first.index_select(0, idx)
        return c

    def scatter_(self, rows, sub: "RWKVState") -> "RWKVState":
        """Writes the rows of `sub` back to the listed rows of this state."""
        idx = torch.as_tensor(list(rows), dtype=torch.long, device=self.wkv.device)
        for a, b in zip((self.wkv, self.tmix_prev, self.cmix_prev), (sub.wkv, sub.tmix_prev, sub.cmix_prev)):
            a.index_copy_(1, idx, b)
        self.v_first.index_copy_(0, idx, sub.v_first)
        return self


def _dt(t: torch.Tensor) -> int:
    if t.dtype == torch.float16:
        return _lib.F16
    if t.dtype == torch.float32:
        return _lib.F32
    raise TypeError(f"low-rank matrices must be fp16 or fp32, got {t.dtype}")


@dataclass
class Proj:
    """A projection on the device: kind "sb6" (K3 qblk, qsqm, ddm; xbits),
    "sym" (qblk, qs, d; bits) or "dense" (w [OUT, IN] fp32).  out_per < OUT:
    a row-concatenated group whose row o uses input row o // out_per."""
    kind: str
    bufs: Tuple[torch.Tensor, ...]
    OUT: int
    IN: int
    bits: int = 4
    xbits: int = 0
    out_per: int = 0

    def __post_init__(self):
        if self.out_per == 0:
            self.out_per = self.OUT


def wkv_chunked_prefers(B: int, T: int, H: int) -> bool:
    """Whether the time-chunked WKV-7 forward beats the step-by-step kernel
    for a [B, T, H] pass on MI355X: the step kernel runs B·H·4 workgroups
    for T steps each, the chunked one B·H·⌈T/32⌉ workgroups and then a scan
    of ⌈T/32⌉ steps, so it wins where B·H is small (measured, chunked vs
    step: B1 T128 H12 15.4 vs 19.4 µs, B1 T128 H64 20.6 vs 22.2, B8 T128 H12
    28.1 vs 33.3, B1 T256 H12 18.3 vs 36.4, B1 T1024 H12 48 vs 139, B1 T8192
    H64 0.77 vs 1.2 ms; B32 T128 H16 loses, 114 vs 63 µs)."""
    return B * H <= 128 and T >= 128


class X070Decoder:
    """Device-resident x070 model (quantised projections + dense parameters)
    and its one-token step.

    dense: the `gg` parameters by the reference's x070 names
    (RwkvqSidecar.buildDenseWeights' dictionary; numpy arrays or tensors);
    proj: world key (X070Shape.projections names) → Proj, or an sb6
    (qblk, qsqm, ddm, OUT, IN) tuple of K3 buffers (xbits from `xbits`).
    The r/k/v projections of a layer run as one fused GEMV when they share
    kind and format."""

    def __init__(self, n_layer: int, n_embd: int, ffn: int, vocab: int, dense: Dict[str, object],
                 proj: Dict[str, object], device, xbits: int = 0):
        self.L, self.D, self.F, self.V = n_layer, n_embd, ffn, vocab
        self.H = n_embd // HEAD
        self.device = torch.empty(0, device=device).device   # concrete index (cuda → cuda:N)
        # one launch for a layer's r/k/v GEMV and low-rank first layers where
        # _fused_rkv_lora allows (bitwise equal to the two launches)
        self.fuse_rkv_lora = True
        # batch 1: the r/k/v + low-rank and ffn key launches form their input
        # rows (layer norm, token shift, lerps) themselves, two launches per
        # layer fewer (bitwise the shift_mix path), where _ln_fused allows
        self.fuse_ln = True
        dev = self.device

        def tens(a) -> torch.Tensor:
            return a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a))

        f32 = lambda a: tens(a).to(device=dev, dtype=torch.float32).reshape(-1).contiguous()

        def lowrank(a) -> torch.Tensor:
            t = tens(a).to(dev).contiguous()
            if t.dtype not in (torch.float16, torch.float32):
                raise TypeError(f"low-rank matrices must be fp16 or fp32, got {t.dtype}")
            return t

        emb = tens(dense["emb.weight"]).to(dev)
        self.emb = emb.contiguous() if emb.dtype in (torch.float16, torch.float32) else emb.float().contiguous()
        self.ln0 = (f32(dense["ln0.weight"]), f32(dense["ln0.bias"]))
        self.ln_out = (f32(dense["ln_out.weight"]), f32(dense["ln_out.bias"]))
        def rank_of(l, nm):
            k = f"blocks.{l}.tmix.{nm}_lora_A.weight"
            return int(tens(dense[k]).shape[0]) if k in dense else None

        # layer 0 has no value-residual branch (RwkvqFullConvert.swift:20-25); its
        # slot in the low-rank buffers keeps the model's v rank, never read
        rv = next((r for r in (rank_of(l, "v") for l in range(n_layer)) if r), 8)
        ranks = (rank_of(0, "w"), rank_of(0, "a"), rv, rank_of(0, "g"))
        self.layers = []
        for l in range(n_layer):
            b, t = f"blocks.{l}.", f"blocks.{l}.tmix."
            has_v = t + "v_lora_A.weight" in dense
            if l > 0 and not has_v:
                raise KeyError(f"{t}v_lora_A.weight: layers above 0 need the value-residual branch")
            A = [lowrank(dense[t + nm + "_lora_A.weight"]) for nm in "wag"]
            dt = A[0].dtype
            A.insert(2, lowrank(dense[t + "v_lora_A.weight"]) if has_v else
                     torch.zeros((rv, n_embd), dtype=dt, device=dev))
            B = [lowrank(dense[t + nm + "_lora_B.weight"]) for nm in "wag"]
            B.insert(2, lowrank(dense[t + "v_lora_B.weight"]) if has_v else
                     torch.zeros((n_embd, rv), dtype=dt, device=dev))
            if tuple(int(x.shape[0]) for x in A) != ranks or any(int(m.shape[1]) != r for m, r in zip(B, ranks)):
                raise ValueError(f"layer {l}: low-rank sizes differ from layer 0's {ranks}")
            lay = {
                "ln1": (f32(dense[b + "ln1.weight"]), f32(dense[b + "ln1.bias"])),
                "ln2": (f32(dense[b + "ln2.weight"]), f32(dense[b + "ln2.bias"])),
                "coef6": torch.stack([f32(dense[t + "x_" + c]) for c in _COEF_ORDER]).contiguous(),
                "ck": f32(dense[b + "cmix.x_k"]),
                "wcat": torch.cat(A, 0).contiguous(),
                "B": B,
                "bias": [f32(dense[t + "w_lora_B.bias"]), f32(dense[t + "a_lora_B.bias"]),
                         f32(dense[t + "v_lora_B.bias"]) if has_v else torch.zeros(n_embd, device=dev)],
                "k_k": f32(dense[t + "k_k"]), "k_a": f32(dense[t + "k_a"]), "r_k": f32(dense[t + "r_k"]),
                "lnx": (f32(dense[t + "ln_x.weight"]), f32(dense[t + "ln_x.bias"])),
            }
            if len({lay["wcat"].dtype} | {m.dtype for m in B}) != 1:
                raise TypeError("low-rank matrices of a layer must share one dtype")
            self.layers.append(lay)
        self.ranks = ranks
        self.proj: Dict[str, object] = {}
        as_proj = lambda v: v if isinstance(v, Proj) else self._sb6(v, xbits)
        for l in range(n_layer):
            keys = [f"blocks.{l}.att.{m}.weight" for m in ("receptance", "key", "value")]
            self.proj[f"blocks.{l}.att.rkv"] = self._group([as_proj(proj[k]) for k in keys])
            for k in (f"blocks.{l}.att.output.weight", f"blocks.{l}.ffn.key.weight", f"blocks.{l}.ffn.value.weight"):
                self.proj[k] = as_proj(proj[k])
        self.proj["head.weight"] = as_proj(proj["head.weight"])
        self._bufs: Optional[dict] = None
        self._tmp: Dict[tuple, torch.Tensor] = {}
        # T16 copies (quant.rwkvq_sb6_t16) of the sb6 projections that take
        # the batched matrix-core GEMV, made with the buffers of a batch size
        self._t16: Dict[int, tuple] = {}
        # (projection, rows, batch_mfma) → (chunk sizes, workspace bytes) or None:
        # the batched-GEMV decision, made once (eager steps pay per ctypes call)
        self._plans: Dict[tuple, Optional[tuple]] = {}
        self._t16p: Dict[int, tuple] = {}   # device addresses of the T16 copies

    @classmethod
    def from_sidecar(cls, sc, device=None, param_dtype=torch.float16) -> "X070Decoder":
        """X070Backbone.load(fromSidecar:) (RwkvqStandaloneLoad.swift:164-194)
        for decoding: the dense body from RwkvqSidecar.build_dense_weights and
        every projection kept in its file layout (sb6 K3 / sym on the GEMV;
        other kinds dequantised once to fp32)."""
        from .quant import RwkvqKind

        device = device or next(iter(sc.arrays.values())).device
        dense = sc.build_dense_weights(param_dtype)
        keys = [f"blocks.{l}.att.{m}.weight" for l in range(sc.n_layer)
                for m in ("receptance", "key", "value", "output")]
        keys += [f"blocks.{l}.ffn.{m}.weight" for l in range(sc.n_layer) for m in ("key", "value")]
        keys.append("head.weight")
        proj = {}
        for k in keys:
            info = sc.tensors.get(k)
            if info is None:
                from .quant import MissingBuffer
                raise MissingBuffer(k, "manifest")
            OUT, IN = info.out_features, info.in_features
            if info.kind == RwkvqKind.sb6:
                proj[k] = Proj("sb6", tuple(sc.arrays[f"{k}::{f}"] for f in ("qblk", "qsqm", "ddm")), OUT, IN,
                               bits=info.bits, xbits=info.xbits)
            elif info.kind == RwkvqKind.sym:
                proj[k] = Proj("sym", tuple(sc.arrays[f"{k}::{f}"] for f in ("qblk", "qs", "d")), OUT, IN,
                               bits=info.bits)
            else:
                proj[k] = Proj("dense", (sc.dequantize(k, torch.float32).contiguous(),), OUT, IN)
        ffn = sc.tensors["blocks.0.ffn.key.weight"].out_features
        return cls(sc.n_layer, sc.n_embd, ffn, sc.vocab_size, dense, proj, device)

    def _sb6(self, t, xbits) -> Proj:
        dev = self.device
        tt = lambda a: (a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a))).to(dev)
        ddm = t[2] if isinstance(t[2], torch.Tensor) else np.ascontiguousarray(t[2]).view(np.uint16)
        return Proj("sb6", (tt(t[0]), tt(t[1]), tt(ddm)), int(t[3]), int(t[4]), bits=4 + xbits, xbits=xbits)

    @staticmethod
    def _group(parts):
        """One fused Proj when the members share kind and format, else the list."""
        p0 = parts[0]
        same = all(p.kind == p0.kind and p.bits == p0.bits and p.xbits == p0.xbits and p.OUT == p0.OUT
                   and p.IN == p0.IN for p in parts)
        if same and p0.kind in ("sb6", "sym"):
            bufs = tuple(torch.cat([p.bufs[i] for p in parts], 0).contiguous() for i in range(3))
            return Proj(p0.kind, bufs, p0.OUT * len(parts), p0.IN, bits=p0.bits, xbits=p0.xbits, out_per=p0.OUT)
        return list(parts)

    def new_state(self, n_rows: int) -> RWKVState:
        return RWKVState(self.L, n_rows, self.D, self.device)

    def _buffers(self, N: int) -> dict:
        if self._bufs is None or self._bufs["N"] != N:
            for q in self.proj.values():
                if self._batch_chunks(q, N) is not None and id(q) not in self._t16:
                    self._t16[id(q)] = Q.rwkvq_sb6_t16(*q.bufs, q.OUT, q.IN)
            dev, D = self.device, self.D
            z = lambda *s: torch.empty(s, dtype=torch.float32, device=dev)
            self._bufs = {"N": N, "x": z(N, D), "xrkv": z(N, 3, D), "xmix": z(N, 4, D), "y_rkv": z(N, 3 * D),
                          "la": z(N, sum(self.ranks)), "tout": z(N, D), "xk": z(N, D), "hk": z(N, self.F),
                          "xo": z(N, D), "xl": z(D), "xl1": z(D), "xl2": z(D), "logits": z(N, self.V)}
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
        _lib.check(L.rwkv_layer_norm(p(self.emb), emb_dt, p(ids), int(self.emb.shape[0]), p(self.ln0[0]),
                                     p(self.ln0[1]), p(x), N, D, LN_EPS, s))
        if self._ln_fused(N):
            for l, lay in enumerate(self.layers):
                self._layer_ln_fused(l, lay, state, bf, s)
            return self._head(bf, N, s)
        for l, lay in enumerate(self.layers):
            _lib.check(L.rwkv_x070_shift_mix(p(x), p(lay["ln1"][0]), p(lay["ln1"][1]), p(state.tmix_prev[l]),
                                             p(lay["coef6"]), 6, p(bf["xrkv"]), p(bf["xmix"]), N, D, LN_EPS, s))
            if not self._rkv_lora(l, lay, bf, N, s):
                self._rkv(l, bf, N, s)
                self._lora_in(l, lay, bf, N, s)
            self._tmix_core(l, lay, state, bf, N, s)
            self._gemv(f"blocks.{l}.att.output.weight", bf["tout"], x, 1, N, s)
            _lib.check(L.rwkv_x070_shift_mix(p(x), p(lay["ln2"][0]), p(lay["ln2"][1]), p(state.cmix_prev[l]),
                                             p(lay["ck"]), 1, p(bf["xk"]), None, N, D, LN_EPS, s))
            self._gemv(f"blocks.{l}.ffn.key.weight", bf["xk"], bf["hk"], 2, N, s)
            self._gemv(f"blocks.{l}.ffn.value.weight", bf["hk"], x, 1, N, s)
        return self._head(bf, N, s)

    def _head(self, bf, N, s) -> torch.Tensor:
        L, p = _lib.lib(), (lambda t: t.data_ptr())
        _lib.check(L.rwkv_layer_norm(p(bf["x"]), _lib.F32, None, 0, p(self.ln_out[0]), p(self.ln_out[1]),
                                     p(bf["xo"]), N, self.D, LN_EPS, s))
        self._gemv("head.weight", bf["xo"], bf["logits"], 0, N, s)
        return bf["logits"]

    def _ln_fused(self, N) -> bool:
        """Batch 1 with every layer's r/k/v group and low-rank first layers
        fused, 4-bit sb6 ffn key / value, and the x070 plans
        (rwkv_x070_ln_fused_applies)."""
        if not (self.fuse_ln and N == 1):
            return False
        for l in range(self.L):
            kv = [self.proj[f"blocks.{l}.ffn.{k}.weight"] for k in ("key", "value")]
            if not (self._fused_rkv_lora(l, N) and all(isinstance(q, Proj) and q.kind == "sb6" and q.xbits == 0
                                                       for q in kv)):
                return False
        return bool(_lib.lib().rwkv_x070_ln_fused_applies(self.D, self.F, 0))

    def _layer_ln_fused(self, l, lay, state, bf, s):
        """One layer of the batch-1 step in five launches: r/k/v + low-rank
        (forming the ln1 / shift rows; ln1 row → xl1), the tmix core (which
        stores xl1 as the next tmix shift row), o_proj + residual, ffn key
        (forming the ln2 / shift row; ln2 row → xl2), ffn value + residual
        (which stores xl2 as the next cmix shift row)."""
        L, p = _lib.lib(), (lambda t: t.data_ptr())
        q = self.proj[f"blocks.{l}.att.rkv"]
        rw, ra, rv, rg = self.ranks
        x = bf["x"]
        _lib.check(L.rwkv_x070_rkv_lora_ln(p(x), p(lay["ln1"][0]), p(lay["ln1"][1]), p(state.tmix_prev[l]),
                                           p(lay["coef6"]), LN_EPS, p(bf["xl1"]), p(q.bufs[0]), p(q.bufs[1]),
                                           p(q.bufs[2]), p(bf["y_rkv"]), self.D, 0, p(lay["wcat"]), _lib.F16,
                                           rw, ra, rv, rg, int(l > 0), p(bf["la"]), s))
        self._tmix_core(l, lay, state, bf, 1, s, shift=(bf["xl1"], state.tmix_prev[l]))
        self._gemv(f"blocks.{l}.att.output.weight", bf["tout"], x, 1, 1, s)
        k = self.proj[f"blocks.{l}.ffn.key.weight"]
        _lib.check(L.rwkv_x070_ffn_key_ln(p(x), p(lay["ln2"][0]), p(lay["ln2"][1]), p(state.cmix_prev[l]),
                                          p(lay["ck"]), LN_EPS, p(bf["xl2"]), p(k.bufs[0]), p(k.bufs[1]),
                                          p(k.bufs[2]), p(bf["hk"]), self.F, self.D, 0, s))
        v = self.proj[f"blocks.{l}.ffn.value.weight"]
        _lib.check(L.rwkv_x070_ffn_value(p(bf["hk"]), p(v.bufs[0]), p(v.bufs[1]), p(v.bufs[2]), p(x), self.D, self.F,
                                         0, p(bf["xl2"]), p(state.cmix_prev[l]), s))

    def launches_per_token(self, N: int = 1) -> int:
        """Kernel launches of one step of N rows: per layer 2 shift_mix +
        lora_in + tmix_core and the projections (one per sb6 / sym GEMV or
        fused group, one or two per chunk of the batched matrix-core GEMV
        (rwkv_sb6_gemv_batch_t16_launches); a dense
        one is the library GEMM plus its epilogue's
        elementwise kernels; r / k / v taken one by one at N > 1 add two
        staging copies each; the r/k/v group and lora_in as one launch where
        _fused_rkv_lora holds), plus emb/ln0, ln_out and the head."""
        def n(q, ep=0, staged=False):
            if isinstance(q, list):
                return sum(n(m, ep, N > 1) for m in q)
            chunks = self._batch_chunks(q, N)
            if chunks is not None:   # one (row-owned) or two (K slices + reduction) per chunk
                L = _lib.lib()
                return sum(int(L.rwkv_sb6_gemv_batch_t16_launches(n, q.OUT, q.IN, q.out_per)) for n in chunks) + \
                    2 * staged
            k = 1 + (1 + 2 * (ep == 2) if q.kind == "dense" else 0)
            return k + 2 * staged
        if self._ln_fused(N):   # r/k/v + low-rank, tmix core, o, ffn key, ffn value
            return sum(4 + n(self.proj[f"blocks.{l}.att.output.weight"], 1) for l in range(self.L)) + 2 + n(
                self.proj["head.weight"])
        # 2 shift_mix + tmix_core + (lora_in and the r/k/v projections, or
        # their one fused launch) + o / ffn key / ffn value
        per_layer = sum((4 if self._fused_rkv_lora(l, N) else 4 + n(self.proj[f"blocks.{l}.att.rkv"])) + sum(
            n(self.proj[f"blocks.{l}.{k}.weight"], ep) for k, ep in (("att.output", 1), ("ffn.key", 2),
                                                                       ("ffn.value", 1)))
            for l in range(self.L))
        return per_layer + 2 + n(self.proj["head.weight"])

    def _fused_rkv_lora(self, l, N) -> bool:
        """The layer's r/k/v GEMV and low-rank first layers run as one launch
        (rwkv_x070_rkv_lora): batch 1, one 4-bit sb6 r/k/v group, fp16
        low-rank matrices."""
        q = self.proj[f"blocks.{l}.att.rkv"]
        return (self.fuse_rkv_lora and N == 1 and isinstance(q, Proj) and q.kind == "sb6" and q.xbits == 0
                and q.out_per < q.OUT and self.layers[l]["wcat"].dtype == torch.float16)

    def _rkv_lora(self, l, lay, bf, N, s) -> bool:
        if not self._fused_rkv_lora(l, N):
            return False
        L, p = _lib.lib(), (lambda t: t.data_ptr())
        q = self.proj[f"blocks.{l}.att.rkv"]
        rw, ra, rv, rg = self.ranks
        _lib.check(L.rwkv_x070_rkv_lora(p(bf["xrkv"]), p(q.bufs[0]), p(q.bufs[1]), p(q.bufs[2]), p(bf["y_rkv"]),
                                        q.OUT, q.IN, q.xbits, q.out_per, p(bf["xmix"]), p(lay["wcat"]), _lib.F16,
                                        rw, ra, rv, rg, int(l > 0), p(bf["la"]), s))
        return True

    def _lora_in(self, l, lay, bf, N, s):
        L, p = _lib.lib(), (lambda t: t.data_ptr())
        rw, ra, rv, rg = self.ranks
        _lib.check(L.rwkv_x070_lora_in(p(bf["xmix"]), p(lay["wcat"]), _dt(lay["wcat"]), rw, ra, rv, rg, int(l > 0),
                                       p(bf["la"]), N, self.D, s))

    def _tmix_core(self, l, lay, state, bf, N, s, shift=None):
        L, p = _lib.lib(), (lambda t: t.data_ptr())
        rw, ra, rv, rg = self.ranks
        wdt = _dt(lay["wcat"])
        Bm = lay["B"]
        _lib.check(L.rwkv_x070_tmix_core(p(bf["y_rkv"]), p(bf["la"]), p(Bm[0]), p(Bm[1]), p(Bm[2]), p(Bm[3]), wdt,
                                         rw, ra, rv, rg, p(lay["bias"][0]), p(lay["bias"][1]), p(lay["bias"][2]),
                                         p(lay["k_k"]), p(lay["k_a"]), p(lay["r_k"]), p(lay["lnx"][0]),
                                         p(lay["lnx"][1]), p(state.v_first), int(l == 0), p(state.wkv[l]),
                                         p(bf["tout"]), N, self.H, LNX_EPS, None if shift is None else p(shift[0]),
                                         None if shift is None else p(shift[1]), s))

    def _gemv(self, key, x, y, ep, N, s):
        self._run(self.proj[key], x, y, ep, N, s)

    # Which sb6 projections of a batch take the matrix-core batched GEMV
    # (within fp32 rounding of each row alone) instead of the one-input
    # arithmetic run over the rows (bitwise each row alone): None = where it
    # is faster and the batch has 5+ rows (quant.rwkvq_sb6_gemv_batch_prefers:
    # K <= 1024, or 16+ rows of any matrix, 8+ of 2^22+ weights, 2^24+),
    # True = wherever it applies (2+ rows), False = never.
    batch_mfma: Optional[bool] = None

    def _batch_ws(self, nbytes: int) -> torch.Tensor:
        """The workspace the batched GEMV and the split long-pass GEMM share
        (their launches are ordered on the stream), grown when a call needs more.
        A grown-out buffer is kept alive (not returned to the caching
        allocator): a HIP graph captured through launch() before the growth
        still holds its address and may be replayed."""
        ws = self._tmp.get("batch_ws")
        if ws is None or ws.numel() < nbytes:
            if ws is not None:
                self._tmp.setdefault("batch_ws_retired", []).append(ws)
            ws = self._tmp["batch_ws"] = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=self.device)
        return ws

    def _batch_chunks(self, q, N: int) -> Optional[List[int]]:
        """Row counts of the rwkv_sb6_gemv_batch launches a projection of N
        rows takes (chunks of at most 32), or None where it keeps the
        one-input kernels."""
        if not isinstance(q, Proj) or q.kind != "sb6" or q.xbits != 0 or N < 2 or self.batch_mfma is False:
            return None
        if self.batch_mfma is None and not Q.rwkvq_sb6_gemv_batch_prefers(N, q.OUT, q.IN):
            return None
        nch = (N + 31) // 32
        sizes = [N // nch + (1 if c < N % nch else 0) for c in range(nch)]
        L = _lib.lib()
        if not all(L.rwkv_sb6_gemv_batch_applies(n, q.OUT, q.IN, 0, q.out_per) for n in set(sizes)):
            return None
        return sizes

    def _batch_plan(self, q, N: int) -> Optional[tuple]:
        """(_batch_chunks, the workspace bytes they need), or None; memoised."""
        key = (id(q), N, self.batch_mfma)
        if key not in self._plans:
            sizes = self._batch_chunks(q, N)
            plan = None
            if sizes is not None:
                L = _lib.lib()
                plan = (sizes, max(int(L.rwkv_sb6_gemv_batch_workspace(n, q.OUT, q.IN, q.out_per)) for n in set(sizes)))
            self._plans[key] = plan
        return self._plans[key]

    def _run_batch(self, q: Proj, x: torch.Tensor, y: torch.Tensor, ep: int, N: int, s) -> bool:
        """rwkv_sb6_gemv_batch_t16 over chunks of at most 32 rows, on the
        projection's T16 copy; False where it does not apply."""
        plan = self._batch_plan(q, N)
        if plan is None:
            return False
        sizes, need = plan
        t16 = self._t16.get(id(q))
        if t16 is None:   # (launch makes them with its buffers, before any capture)
            t16 = self._t16[id(q)] = Q.rwkvq_sb6_t16(*q.bufs, q.OUT, q.IN)
        tp = self._t16p.get(id(q))
        if tp is None:
            tp = self._t16p[id(q)] = tuple(b.data_ptr() for b in t16)
        L = _lib.lib()
        K = q.OUT // q.out_per
        ws = self._batch_ws(need)
        if not x.is_contiguous():
            x = x.contiguous()
        # chunk n0 starts at input row n0: plain pointer offsets (x [N, K, IN],
        # y [N, OUT] fp32, contiguous), no views per call
        xp, yp, wp, wn = x.data_ptr(), y.data_ptr(), ws.data_ptr(), ws.numel()
        n0 = 0
        for n in sizes:
            _lib.check(L.rwkv_sb6_gemv_batch_t16(xp + 4 * n0 * K * q.IN, n, *tp, yp + 4 * n0 * q.OUT, q.OUT, q.IN,
                                                 q.out_per, ep, wp, wn, s))
            n0 += n
        return True

    def _run(self, q: Proj, x: torch.Tensor, y: torch.Tensor, ep: int, N: int, s) -> None:
        """y = ep(x · Wᵀ): ep 0 store, 1 add into y, 2 relu² (rwkv_*_gemv_ep)."""
        L = _lib.lib()
        if self._run_batch(q, x, y, ep, N, s):
            return
        if q.kind == "sb6":
            if q.out_per < q.OUT:
                if ep != 0:
                    raise ValueError("a fused group stores its result (epilogue 0)")
                _lib.check(L.rwkv_sb6_gemv_fused(x.data_ptr(), N, *[b.data_ptr() for b in q.bufs], y.data_ptr(),
                                                 q.OUT, q.IN, q.xbits, q.out_per, s))
            else:
                _lib.check(L.rwkv_sb6_gemv_ep(x.data_ptr(), N, *[b.data_ptr() for b in q.bufs], y.data_ptr(),
                                              q.OUT, q.IN, q.xbits, ep, s))
        elif q.kind == "sym":
            if q.out_per < q.OUT:
                if ep != 0:
                    raise ValueError("a fused group stores its result (epilogue 0)")
                _lib.check(L.rwkv_sym_gemv(x.data_ptr(), N, *[b.data_ptr() for b in q.bufs], y.data_ptr(),
                                           q.OUT, q.IN, q.bits, q.out_per, s))
            else:
                _lib.check(L.rwkv_sym_gemv_ep(x.data_ptr(), N, *[b.data_ptr() for b in q.bufs], y.data_ptr(),
                                              q.OUT, q.IN, q.bits, ep, s))
        else:   # dense: the library GEMM on torch's current stream
            if s != torch.cuda.current_stream(self.device).cuda_stream:
                raise ValueError("dense projections run on the current stream only")
            tmp = self._tmp.get((id(q), N))
            if tmp is None:
                tmp = self._tmp[(id(q), N)] = torch.empty((N, q.OUT), dtype=torch.float32, device=self.device)
            torch.mm(x.reshape(N, q.IN), q.bufs[0].t(), out=tmp)
            yv = y.reshape(N, q.OUT)
            if ep == 1:
                yv.add_(tmp)
            elif ep == 2:
                torch.relu_(tmp)
                yv.copy_(tmp.square_())
            else:
                yv.copy_(tmp)

    def _rkv(self, l, bf, N, s):
        """r / k / v projections of layer l into y_rkv [N, 3D]: one fused GEMV,
        or the three matrices one by one (through contiguous staging rows
        when N > 1)."""
        q = self.proj[f"blocks.{l}.att.rkv"]
        if isinstance(q, Proj):
            self._run(q, bf["xrkv"], bf["y_rkv"], 0, N, s)
            return
        D = self.D
        for k, qk in enumerate(q):
            if N == 1:
                self._run(qk, bf["xrkv"][0, k], bf["y_rkv"][0, k * D:(k + 1) * D], 0, 1, s)
            else:
                xi = self._tmp.setdefault(("rkv_x", N), torch.empty((N, D), device=self.device))
                yi = self._tmp.setdefault(("rkv_y", N), torch.empty((N, D), device=self.device))
                xi.copy_(bf["xrkv"][:, k])
                self._run(qk, xi, yi, 0, N, s)
                bf["y_rkv"][:, k * D:(k + 1) * D].copy_(yi)

    def step(self, ids, state: RWKVState) -> torch.Tensor:
        """X070Backbone.step (X070Generation.swift:437-474): token ids [N]
        (ints or a device int32 tensor) → logits [N, vocab] (a new tensor);
        `state` advances by one token per row."""
        if not isinstance(ids, torch.Tensor):
            ids = torch.tensor(np.asarray(ids, np.int32).reshape(-1), device=self.device)
        return self.launch(ids.to(device=self.device, dtype=torch.int32).reshape(-1), state).clone()

    def step_batch(self, ids, state: RWKVState) -> torch.Tensor:
        """stepBatch (BatchGenerate.swift:56-63): one token per row of `state`."""
        if len(ids) != state.n_rows:
            raise ValueError(f"step_batch: {len(ids)} tokens for a batch of {state.n_rows}")
        return self.step(ids, state)

    def prefill_batch(self, prompts, base_dtype=torch.float16, short_rows: int = 0,
                      wkv_chunked: Optional[bool] = None, graph: bool = False) -> Tuple[torch.Tensor, RWKVState]:
        """prefillBatch (BatchGenerate.swift:37-53): every prompt in one
        parallel pass — right padding to the longest prompt, a mask that makes
        the pad steps neutral for the recurrence, each row's shift state taken
        at its last real token — returning the logits [B, vocab] of each
        prompt's last token and the batch state.  Per layer (rwkvTmixForward /
        rwkvCmixForward, RWKVBlock.swift:163-307): ln1 + token shift + lerps
        over the sequence, the r/k/v projections, the low-rank branches, the
        time-mix arithmetic with the pad mask, one WKV-7 launch for the whole
        sequence from the row's state, the tail, o_proj + residual, ln2 +
        shift, the FFN.  Projections (baseProj, X070Backbone.swift:676-746):
        with `base_dtype` fp16, B·T rows above `short_rows` take the fp16 long
        pass on the matrix cores (rwkv_sb6_gemm for 4-bit sb6; dequantise +
        library GEMM otherwise), the others the fp32 GEMV; with fp32 every
        projection is the fp32 GEMV.  The head is the GEMV (decode: true).
        The WKV-7 pass runs in 32-token chunks in parallel over time
        (rwkv_wkv7_seq_fwd_chunked) when `wkv_chunked` is True, or when it is
        None and the pass has few (batch, head) rows and a long T
        (wkv_chunked_prefers); otherwise step by step (rwkv_wkv7_seq_fwd).
        `graph`: the pass is captured into a HIP graph once per (B, T, kind)
        and replayed (one host call instead of ~25 launches per layer; the
        same launches, so the same results)."""
        if len(prompts) == 0:
            raise ValueError("prefill_batch: no prompts")
        if any(len(p) == 0 for p in prompts):
            raise ValueError("prefill_batch: empty prompt")
        if base_dtype not in (torch.float16, torch.float32):
            raise ValueError(f"prefill_batch: base dtype {base_dtype} (float16 or float32)")
        B, T = len(prompts), max(len(p) for p in prompts)
        M = B * T
        long = base_dtype == torch.float16 and M > short_rows
        # the long pass's kernels take up to 2^24 rows; the fp32 GEMV's
        # batched plan (short passes and the fp32 base) 65535
        most = (1 << 24) if long else 65535
        if M > most:
            raise ValueError(f"prefill_batch: {M} rows in one pass (at most {most})")
        dev = self.device
        ids = np.zeros((B, T), np.int32)
        for i, p in enumerate(prompts):
            ids[i, :len(p)] = np.asarray(p, np.int32)
        lens = [len(p) for p in prompts]
        last = [i * T + n - 1 for i, n in enumerate(lens)]
        # the chunk transforms' workspace (48 KiB per (row, head, chunk)) at most 16 GiB
        chunked = (wkv_chunked_prefers(B, T, self.H) and B * self.H * ((T + 31) // 32) * 49152 <= (16 << 30)
                   if wkv_chunked is None else bool(wkv_chunked))
        if graph:
            return self._prefill_graphed(ids, lens, last, B, T, long, chunked)
        ids_t = torch.from_numpy(ids.reshape(-1)).to(dev)
        len_t = torch.tensor(lens, dtype=torch.int32, device=dev)
        last_t = torch.tensor(last, dtype=torch.int32, device=dev)
        state = self.new_state(B)
        logits = torch.empty((B, self.V), dtype=torch.float32, device=dev)
        bf = self._prefill_setup(B, T, long, chunked)
        self._prefill_run(bf, ids_t, len_t, last_t, state, logits, B, T, long, torch.cuda.current_stream(dev).cuda_stream)
        return logits, state

    def _prefill_setup(self, B: int, T: int, long: bool, chunked: bool) -> dict:
        """The pass's buffers (and the chunked WKV-7 workspace), made before
        any launch so the pass can be captured."""
        bf = self._prefill_buffers(B * T, long)
        if chunked:
            need = int(_lib.lib().rwkv_wkv7_chunked_workspace(B, T, self.H))
            if bf.get("wkv_ws") is None or bf["wkv_ws"].numel() < need:
                bf["wkv_ws"] = torch.empty(need, dtype=torch.uint8, device=self.device)
        if bf.get("xo") is None or bf["xo"].shape[0] != B:
            bf["xo"] = torch.empty((B, self.D), dtype=torch.float32, device=self.device)
        bf["chunked"] = chunked
        return bf

    def _prefill_run(self, bf, ids_t, len_t, last_t, state, logits, B, T, long, s) -> None:
        """The device work of one parallel pass: every launch on stream s, no
        allocation and no host synchronisation."""
        M, D = B * T, self.D
        L, p = _lib.lib(), (lambda t: t.data_ptr())
        x = bf["x"]
        emb_dt = _lib.F16 if self.emb.dtype == torch.float16 else _lib.F32
        _lib.check(L.rwkv_layer_norm(p(self.emb), emb_dt, p(ids_t), int(self.emb.shape[0]), p(self.ln0[0]),
                                     p(self.ln0[1]), p(x), M, D, LN_EPS, s))
        for l in range(self.L):
            self._prefill_layer(l, state, bf, len_t, B, T, long, s)
        xo = bf["xo"]
        _lib.check(L.rwkv_layer_norm(p(x), _lib.F32, p(last_t), M, p(self.ln_out[0]), p(self.ln_out[1]), p(xo),
                                     B, D, LN_EPS, s))
        self._gemv("head.weight", xo, logits, 0, B, s)

    def _prefill_graphed(self, ids, lens, last, B, T, long, chunked):
        """prefill_batch replayed from a HIP graph captured once per (B, T,
        pass kind): the prompts' ids, lengths and last-token rows are copied
        into the graph's own input buffers, the state starts from zeros inside
        the graph, and the logits and state are returned as copies."""
        key = ("prefill_graph", B, T, long, chunked)
        gr = self._tmp.get(key)
        dev = self.device
        if gr is None:
            gr = {"ids": torch.zeros(B * T, dtype=torch.int32, device=dev),
                  "len": torch.ones(B, dtype=torch.int32, device=dev),
                  "last": torch.zeros(B, dtype=torch.int32, device=dev),
                  "state": self.new_state(B),
                  "logits": torch.empty((B, self.V), dtype=torch.float32, device=dev)}
        gr["ids"].copy_(torch.from_numpy(ids.reshape(-1)))
        gr["len"].copy_(torch.tensor(lens, dtype=torch.int32))
        gr["last"].copy_(torch.tensor(last, dtype=torch.int32))
        st = gr["state"]

        def run(s):
            for t in (st.wkv, st.tmix_prev, st.cmix_prev, st.v_first):
                t.zero_()
            self._prefill_run(bf, gr["ids"], gr["len"], gr["last"], st, gr["logits"], B, T, long, s)

        if "graph" not in gr:
            # a copy of the buffer table: the graph keeps the tensors it was
            # captured with alive even when a later eager pass replaces them
            bf = dict(self._prefill_setup(B, T, long, chunked))
            side = torch.cuda.Stream(device=dev)
            side.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(side):
                run(side.cuda_stream)   # eager once: plans and buffers exist before capture
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=side):
                    run(torch.cuda.current_stream(dev).cuda_stream)
            torch.cuda.current_stream(dev).wait_stream(side)
            gr["graph"], gr["bf"] = g, bf
            self._tmp[key] = gr
        gr["graph"].replay()
        return gr["logits"].clone(), st.clone()

    def _prefill_buffers(self, M: int, long: bool) -> dict:
        key = ("prefill", M, long)
        bf = self._tmp.get(key)
        if bf is None:
            dev, D, F = self.device, self.D, self.F
            z = lambda *sh, dt=torch.float32: torch.empty(sh, dtype=dt, device=dev)
            bf = {"x": z(M, D), "xl": z(M, D), "mix": z(6, M, D), "y_rkv": z(M, 3 * D), "v_first": z(M, D),
                  "ww": z(M, D), "aa": z(M, D), "vv": z(M, D), "gate": z(M, D), "wkv": z(M, D), "tout": z(M, D)}
            for n in ("r", "w", "k", "v", "a", "b", "kb"):
                bf[n] = z(M, D)
            bf["rkv_in"] = z(3, M, D, dt=torch.float16) if long else z(M, 3, D)
            if long:   # the tail's output in the fp16 the o_proj long pass reads
                bf["tout"] = z(M, D, dt=torch.float16)
            bf["xk"] = z(M, D, dt=torch.float16) if long else z(M, D)
            bf["hk"] = z(M, F, dt=torch.float16) if long else z(M, F)
            bf["la_seq"] = z(M, sum(self.ranks))
            self._tmp = {k: v for k, v in self._tmp.items() if not (isinstance(k, tuple) and k[0] == "prefill")}
            self._tmp[key] = bf
        return bf

    def _lowrank_f32(self, l: int) -> list:
        """The layer's low-rank matrices in fp32 (the file's fp16 values widen
        exactly): the parallel pass multiplies fp32 activations by them
        without narrowing (MLX promotes the fp16 weight, RWKVBlock.swift:185-226)."""
        key = ("lowrank32", l)
        m = self._tmp.get(key)
        if m is None:
            lay = self.layers[l]
            rw, ra, rv, rg = self.ranks
            A = lay["wcat"].float()
            m = [A[:rw], A[rw:rw + ra], A[rw + ra:rw + ra + rv], A[rw + ra + rv:]] + [t.float() for t in lay["B"]]
            self._tmp[key] = m
        return m

    def _prefill_layer(self, l, state, bf, len_t, B, T, long, s):
        L, p = _lib.lib(), (lambda t: t.data_ptr())
        D, H, F, M = self.D, self.H, self.F, B * T
        lay = self.layers[l]
        x, xl, mix = bf["x"], bf["xl"], bf["mix"]
        # ── time mix ──
        _lib.check(L.rwkv_layer_norm(p(x), _lib.F32, None, 0, p(lay["ln1"][0]), p(lay["ln1"][1]), p(xl), M, D,
                                     LN_EPS, s))
        rkv_in = bf["rkv_in"]
        if long:   # r/k/v inputs fp16 [3, M, D] for the GEMM
            y0 = (rkv_in, _lib.F16, D, M * D)
        else:      # fp32 [M, 3, D] for the fused GEMV
            y0 = (rkv_in, _lib.F32, 3 * D, D)
        # the carried shift state is updated in place
        _lib.check(L.rwkv_x070_seq_shift_mix(p(xl), p(state.tmix_prev[l]), p(state.tmix_prev[l]), p(len_t),
                                             p(lay["coef6"]), 6, 3, p(y0[0]), y0[1], y0[2], y0[3], p(mix), D, M * D,
                                             2, B, T, D, s))
        self._prefill_proj(self.proj[f"blocks.{l}.att.rkv"], rkv_in, bf["y_rkv"], 0, M, long, s)
        rw, ra, rv, rg = self.ranks
        wdt = _dt(lay["wcat"])
        if all(r % 16 == 0 for r in self.ranks) and D % 16 == 0 and (
                M * D <= SEQ_LORA_MAX_MD or L.rwkv_x070_seq_lora_split(M, D, wdt, rw, ra, rv, rg)):
            # the four low-rank branches on the matrix cores (two launches;
            # long passes with fp16 matrices as two fp16 parts per activation)
            Bm = lay["B"]
            _lib.check(L.rwkv_x070_seq_lora(p(mix), M, D, p(lay["wcat"]), p(Bm[0]), p(Bm[1]), p(Bm[2]), p(Bm[3]),
                                            wdt, rw, ra, rv, rg, int(l > 0), p(bf["la_seq"]),
                                            p(bf["ww"]), p(bf["aa"]), p(bf["vv"]), p(bf["gate"]), s))
        else:   # long passes with fp32 matrices (or ranks the kernels do not take): the library's fp32 GEMM
            Aw, Aa, Av, Ag, Bw, Ba, Bv, Bg = self._lowrank_f32(l)
            # mix rows: r, k, v, w, a, g
            torch.mm(torch.tanh(torch.mm(mix[3], Aw.t())), Bw.t(), out=bf["ww"])
            torch.mm(torch.mm(mix[4], Aa.t()), Ba.t(), out=bf["aa"])
            if l > 0:
                torch.mm(torch.mm(mix[2], Av.t()), Bv.t(), out=bf["vv"])
            torch.mm(torch.sigmoid(torch.mm(mix[5], Ag.t())), Bg.t(), out=bf["gate"])
        bias = lay["bias"]
        _lib.check(L.rwkv_x070_seq_tmix_pre(p(bf["y_rkv"]), p(bf["ww"]), p(bf["aa"]), p(bf["vv"]) if l > 0 else None,
                                            p(bias[0]), p(bias[1]), p(bias[2]) if l > 0 else None, p(lay["k_k"]),
                                            p(lay["k_a"]), p(bf["v_first"]), int(l == 0), p(len_t), p(bf["r"]),
                                            p(bf["w"]), p(bf["k"]), p(bf["v"]), p(bf["a"]), p(bf["b"]), p(bf["kb"]),
                                            B, T, H, s))
        st = state.wkv[l]
        if bf["chunked"]:
            ws = bf["wkv_ws"]
            _lib.check(L.rwkv_wkv7_seq_fwd_chunked(p(bf["r"]), p(bf["w"]), p(bf["k"]), p(bf["v"]), p(bf["a"]),
                                                   p(bf["b"]), _lib.F32, p(st), p(bf["wkv"]), p(st), B, T, H,
                                                   p(ws), ws.numel(), s))
        else:
            _lib.check(L.rwkv_wkv7_seq_fwd(p(bf["r"]), p(bf["w"]), p(bf["k"]), p(bf["v"]), p(bf["a"]), p(bf["b"]),
                                           _lib.F32, p(st), p(bf["wkv"]), p(st), B, T, H, s))
        tdt = _lib.F16 if bf["tout"].dtype == torch.float16 else _lib.F32
        _lib.check(L.rwkv_wkv_tail_to(p(bf["wkv"]), p(bf["r"]), p(bf["kb"]), p(bf["v"]), p(lay["r_k"]),
                                      p(lay["lnx"][0]), p(lay["lnx"][1]), p(bf["gate"]), p(bf["tout"]), tdt, M, H,
                                      HEAD, LNX_EPS, s))
        self._prefill_proj(self.proj[f"blocks.{l}.att.output.weight"], bf["tout"], x, 1, M, long, s)
        # ── channel mix ──
        _lib.check(L.rwkv_layer_norm(p(x), _lib.F32, None, 0, p(lay["ln2"][0]), p(lay["ln2"][1]), p(xl), M, D,
                                     LN_EPS, s))
        xk, hk = bf["xk"], bf["hk"]
        _lib.check(L.rwkv_x070_seq_shift_mix(p(xl), p(state.cmix_prev[l]), p(state.cmix_prev[l]), p(len_t),
                                             p(lay["ck"]), 1, 1, p(xk), _lib.F16 if long else _lib.F32, D, M * D,
                                             None, 0, 0, 0, B, T, D, s))
        self._prefill_proj(self.proj[f"blocks.{l}.ffn.key.weight"], xk, hk, 2, M, long, s)
        self._prefill_proj(self.proj[f"blocks.{l}.ffn.value.weight"], hk, x, 1, M, long, s)

    def _prefill_proj(self, q, x, y, ep, M, long, s):
        """A projection of the parallel pass: ep 0 store, 1 add into y, 2
        relu²; long passes through the fp16 base (fp16 inputs / relu² output
        where the buffers are fp16), short ones through the fp32 GEMV."""
        if not long:
            if isinstance(q, list):   # r / k / v one by one: x [M, 3, D] → y [M, 3D]
                for k, qk in enumerate(q):
                    xi = x[:, k].contiguous()
                    yi = torch.empty((M, qk.OUT), dtype=torch.float32, device=self.device)
                    self._run(qk, xi, yi, 0, M, s)
                    y[:, k * qk.OUT:(k + 1) * qk.OUT].copy_(yi)
                return
            self._run(q, x, y, ep, M, s)
            return
        parts = q if isinstance(q, list) else [q]
        G = len(parts) if isinstance(q, list) else (q.OUT // q.out_per)
        xdt = _lib.F16 if x.dtype == torch.float16 else _lib.F32
        xs = x.reshape(G, M, -1) if G > 1 else x.reshape(1, M, -1)
        ldy = y.shape[-1]
        # the matrix-core long pass (rwkv_sb6_gemm / rwkv_sym_gemm) for every
        # sb6 / sym matrix it takes: a fused group in one launch, the members
        # of an unfused r/k/v list each into its columns of y
        if not isinstance(q, list) and self._long_gemm(q, xs[0].data_ptr(), xdt, M, y.data_ptr(), ldy, ep, s):
            return
        col, rest = 0, []
        for g, qq in enumerate(self._split_group(q)):
            if not (isinstance(q, list) and self._long_gemm(qq, xs[g].data_ptr(), xdt, M,
                                                           y.data_ptr() + y.element_size() * col, ldy, ep, s)):
                rest.append((g, col, qq))
            col += qq.OUT
        # other layouts: the reference's long pass — the weight in fp16, then
        # the fp16 matmul (rwkv_f16_gemm where it takes the shape)
        from .quant import rwkvq_dequant_dense, rwkvq_dequant_sym
        L = _lib.lib()
        for g, col, qq in rest:
            if qq.kind == "sb6":
                W = rwkvq_dequant_dense(*qq.bufs, qq.OUT, qq.IN, 8, qq.xbits, torch.float16)
            elif qq.kind == "sym":
                W = rwkvq_dequant_sym(*qq.bufs, qq.OUT, qq.IN, qq.bits, torch.float16)
            else:
                W = qq.bufs[0].to(torch.float16).contiguous()
            x16 = xs[g].to(torch.float16).contiguous()
            if L.rwkv_f16_gemm_applies(M, qq.OUT, qq.IN, qq.OUT):
                _lib.check(L.rwkv_f16_gemm(x16.data_ptr(), M, qq.IN, M * qq.IN, W.data_ptr(),
                                           y.data_ptr() + y.element_size() * col, ldy, qq.OUT, qq.IN, qq.OUT, ep, s))
                continue
            prod = torch.mm(x16, W.t()).float()
            dst = y[:, col:col + qq.OUT] if y.dim() == 2 else y
            if ep == 0:
                dst.copy_(prod)
            elif ep == 1:
                dst.add_(prod)
            else:
                dst.copy_(torch.relu(prod).square_().to(dst.dtype))

    def _long_gemm(self, q, xp, xdt, M, yp, ldy, ep, s) -> bool:
        """One matrix (group) of the long pass on the matrix cores, when the
        kernels take its layout; False otherwise (nothing launched).  Shapes
        with few output tiles split their K sum in the shared workspace."""
        L = _lib.lib()
        if q.kind == "sb6" and L.rwkv_sb6_gemm_applies(q.OUT, q.IN, q.xbits, q.out_per):
            entry, bits = L.rwkv_sb6_gemm, q.xbits
        elif q.kind == "sym" and L.rwkv_sym_gemm_applies(q.OUT, q.IN, q.bits, q.out_per):
            entry, bits = L.rwkv_sym_gemm, q.bits
        else:
            return False
        need = int(L.rwkv_quant_gemm_workspace(M, q.OUT, q.IN))
        ws = self._batch_ws(need).data_ptr() if need else None
        _lib.check(entry(xp, xdt, M, q.IN, M * q.IN, q.bufs[0].data_ptr(), q.bufs[1].data_ptr(), q.bufs[2].data_ptr(),
                         yp, ldy, q.OUT, q.IN, bits, q.out_per, ep, ws, need, s))
        return True

    @staticmethod
    def _split_group(q):
        """The member matrices of a projection (a fused group's row views)."""
        if isinstance(q, list):
            return q
        if q.out_per == q.OUT:
            return [q]
        K = q.OUT // q.out_per
        out = []
        for g in range(K):
            rows = slice(g * q.out_per, (g + 1) * q.out_per)
            out.append(Proj(q.kind, tuple(b[rows] for b in q.bufs), q.out_per, q.IN, bits=q.bits, xbits=q.xbits))
        return out

    def generate_batch(self, prompts, max_tokens: int, stop_tokens=()) -> List[List[int]]:
        """generateBatch (BatchGenerate.swift:71-116) with the greedy choice
        (the first largest logit; greedy does not depend on the per-row seed):
        the continuations of several prompts in one batch.  A row that emits a
        stop token keeps it as its last token and leaves the batch (its state
        rows are gathered out); every row stops at `max_tokens`.  Stop strings
        need a tokenizer and are not part of this path."""
        if max_tokens < 0:
            raise ValueError("generate_batch: max_tokens < 0")
        B = len(prompts)
        produced: List[List[int]] = [[] for _ in range(B)]
        if B == 0 or max_tokens == 0:
            return produced
        stops = {int(t) for t in stop_tokens}
        logits, state = self.prefill_batch(prompts)
        alive = list(range(B))
        for _ in range(max_tokens):
            ids = torch.argmax(logits, dim=1).cpu().tolist()
            nxt, keep = [], []
            for row, i in enumerate(alive):
                produced[i].append(int(ids[row]))
                if ids[row] in stops:
                    continue
                nxt.append(int(ids[row]))
                keep.append(row)
            if not keep:
                break
            if len(keep) < len(alive):
                state = state.gather(keep)
                alive = [alive[r] for r in keep]
            if len(produced[alive[0]]) >= max_tokens:
                break
            logits = self.step(nxt, state)
        return produced

