"""RWKVKernel on MI355X: the Swift module's public API over the HIP C ABI.

Same names (snake_case), argument meaning and shapes as
Sources/RWKVKernel/*.swift; tensors are torch tensors on a ROCm device and
every computation runs in libswiftrwkv_hip.so.  Preconditions that trap in
the reference raise ValueError here (the C ABI returns a status instead).

Module-level switches mirror the reference's process globals:
  wkv7_whole_sequence_forward (WKV7.swift:178), wkv7_backward_v2 and
  wkv7_keep_forward_outputs (WKV7Train.swift:343,354).
Launch counters (WKV7.swift:181, WKV7Train.swift:358) come from the library.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

WKV7_HEAD_SIZE = 64   # WKV7.swift:7
WKV7_CHUNK = 16       # WKV7.swift:8

wkv7_whole_sequence_forward = True
wkv7_backward_v2 = True
wkv7_keep_forward_outputs = True

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous with a 16-byte aligned base (vector and scalar loads assume it)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _prep(xs, ndim_ok=(4,)):
    """Common dtype (the inputs' own if shared and supported, else fp32),
    contiguous, on one ROCm device."""
    dev = xs[0].device
    if dev.type != "cuda":
        raise ValueError(f"WKV-7 inputs must live on a ROCm device, got {dev}")
    shape = xs[0].shape
    for x in xs:
        if x.shape != shape:
            raise ValueError(f"WKV-7 inputs disagree in shape: {tuple(x.shape)} vs {tuple(shape)}")
        if x.device != dev:
            raise ValueError("WKV-7 inputs on different devices")
    if xs[0].dim() not in ndim_ok:
        raise ValueError(f"WKV-7 inputs must have rank {ndim_ok}, got {tuple(shape)}")
    dts = {x.dtype for x in xs}
    only = next(iter(dts))
    dt = only if len(dts) == 1 and only in _DT else torch.float32
    return [_aligned(x.to(dt)) for x in xs], _DT[dt]


def _state(h: Optional[torch.Tensor], shape, dev) -> Optional[torch.Tensor]:
    if h is None:
        return None
    if tuple(h.shape) != tuple(shape):
        raise ValueError(f"hIn {tuple(h.shape)} must be [B,H,D,D] = {list(shape)}")
    return _aligned(h.to(device=dev, dtype=torch.float32))


# ───────────────────────────── frozen forward ─────────────────────────────

def wkv7_sequence_forward(r, w, k, v, a, b, h_in=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Whole sequence in one launch (WKV7.swift:242-264). Inputs [B,T,H,64],
    h_in [B,H,64,64] or None (zeros).  Returns (out [B,T,H,64] f32, h_out)."""
    (r, w, k, v, a, b), dt = _prep([r, w, k, v, a, b])
    B, T, H, D = r.shape
    if T < 1:
        raise ValueError(f"T ({T}) must be >= 1")
    if D != WKV7_HEAD_SIZE:
        raise ValueError(f"D ({D}) must equal HEAD_SIZE {WKV7_HEAD_SIZE}")
    h = _state(h_in, (B, H, D, D), r.device)
    out = torch.empty((B, T, H, D), dtype=torch.float32, device=r.device)
    h_out = torch.empty((B, H, D, D), dtype=torch.float32, device=r.device)
    _lib.call("rwkv_wkv7_seq_fwd", _ptr(r), _ptr(w), _ptr(k), _ptr(v), _ptr(a), _ptr(b), dt, _ptr(h),
              _ptr(out), _ptr(h_out), B, T, H, _stream(r))
    return out, h_out


def wkv7_chunked_workspace_bytes(B: int, T: int, H: int) -> int:
    """Device workspace the time-chunked forward needs (48 KiB per 32 tokens
    per head)."""
    return int(_lib.lib().rwkv_wkv7_chunked_workspace(B, T, H))


def wkv7_sequence_forward_chunked(r, w, k, v, a, b, h_in=None,
                                  workspace: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """The whole-sequence forward of wkv7_sequence_forward (WKV7.swift:242-264)
    computed in 32-token chunks, in parallel over the chunks: for prefill with
    few (batch, head) rows.  Same inputs and outputs; agrees with the
    step-by-step kernel to fp32 rounding (not bitwise).  `workspace` is an
    optional uint8 device buffer of at least wkv7_chunked_workspace_bytes."""
    (r, w, k, v, a, b), dt = _prep([r, w, k, v, a, b])
    B, T, H, D = r.shape
    if T < 1:
        raise ValueError(f"T ({T}) must be >= 1")
    if D != WKV7_HEAD_SIZE:
        raise ValueError(f"D ({D}) must equal HEAD_SIZE {WKV7_HEAD_SIZE}")
    h = _state(h_in, (B, H, D, D), r.device)
    need = wkv7_chunked_workspace_bytes(B, T, H)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=r.device)
    elif workspace.device != r.device or workspace.numel() * workspace.element_size() < need \
            or not workspace.is_contiguous() or workspace.data_ptr() % 16:
        raise ValueError(f"workspace must be a contiguous, 16-byte aligned buffer of >= {need} bytes on {r.device}")
    out = torch.empty((B, T, H, D), dtype=torch.float32, device=r.device)
    h_out = torch.empty((B, H, D, D), dtype=torch.float32, device=r.device)
    _lib.call("rwkv_wkv7_seq_fwd_chunked", _ptr(r), _ptr(w), _ptr(k), _ptr(v), _ptr(a), _ptr(b), dt, _ptr(h),
              _ptr(out), _ptr(h_out), B, T, H, _ptr(workspace), workspace.numel() * workspace.element_size(),
              _stream(r))
    return out, h_out


def wkv7_chunk_forward(r, w, k, v, a, b, h_in) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One 16-token chunk (WKV7.swift:64-82): (out, h_out, sa_out)."""
    (r, w, k, v, a, b), dt = _prep([r, w, k, v, a, b])
    B, T, H, D = r.shape
    if T != WKV7_CHUNK:
        raise ValueError(f"T ({T}) must equal CHUNK {WKV7_CHUNK}")
    if D != WKV7_HEAD_SIZE:
        raise ValueError(f"D ({D}) must equal HEAD_SIZE {WKV7_HEAD_SIZE}")
    h = _state(h_in, (B, H, D, D), r.device)
    if h is None:
        raise ValueError("wkv7_chunk_forward needs an explicit state")
    out = torch.empty((B, T, H, D), dtype=torch.float32, device=r.device)
    sa = torch.empty_like(out)
    h_out = torch.empty((B, H, D, D), dtype=torch.float32, device=r.device)
    _lib.call("rwkv_wkv7_chunk_fwd", _ptr(r), _ptr(w), _ptr(k), _ptr(v), _ptr(a), _ptr(b), dt, _ptr(h),
              _ptr(out), _ptr(h_out), _ptr(sa), B, T, H, _stream(r))
    return out, h_out, sa


def wkv7_forward_chunked(r, w, k, v, a, b, h_in=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """The same pass cut into CHUNK-token launches (WKV7.swift:107-140); the
    tail is padded with neutral steps w = 1, r = k = v = a = b = 0."""
    B, T, H, D = r.shape
    h = h_in if h_in is not None else torch.zeros((B, H, D, D), dtype=torch.float32, device=r.device)
    outs = []
    for start in range(0, T, WKV7_CHUNK):
        end = min(start + WKV7_CHUNK, T)
        cl = end - start

        def sl(x, val):
            c = x[:, start:end]
            if cl < WKV7_CHUNK:
                pad = torch.full((B, WKV7_CHUNK - cl, H, D), val, dtype=c.dtype, device=c.device)
                c = torch.cat([c, pad], dim=1)
            return c

        oc, h, _ = wkv7_chunk_forward(sl(r, 0.0), sl(w, 1.0), sl(k, 0.0), sl(v, 0.0), sl(a, 0.0), sl(b, 0.0), h)
        outs.append(oc[:, :cl])
    return torch.cat(outs, dim=1), h


def wkv7_forward_with_state(r, w, k, v, a, b, h_in=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """WKV7.swift:96-103: whole-sequence launch unless the switch says chunked."""
    if wkv7_whole_sequence_forward:
        return wkv7_sequence_forward(r, w, k, v, a, b, h_in)
    return wkv7_forward_chunked(r, w, k, v, a, b, h_in)


def wkv7_forward(r, w, k, v, a, b) -> torch.Tensor:
    """Zero initial state, final state dropped (WKV7.swift:143-148)."""
    return wkv7_forward_with_state(r, w, k, v, a, b, None)[0]


def wkv7_sequence_launches() -> int:
    c = _lib.counters()
    return c["seq_fwd"] + c["seq_chunked"]


# ───────────────────────────── training (autograd) ─────────────────────────────

def _train_forward(ins, dt, h0):
    r, w, k, v, a, b = ins
    B, T, H, D = r.shape
    out = torch.empty((B, T, H, D), dtype=torch.float32, device=r.device)
    sa = torch.empty_like(out)
    h_out = torch.empty((B, H, D, D), dtype=torch.float32, device=r.device)
    ck = torch.empty((B, H, T // WKV7_CHUNK, D, D), dtype=torch.float32, device=r.device)
    _lib.call("rwkv_wkv7_train_fwd", _ptr(r), _ptr(w), _ptr(k), _ptr(v), _ptr(a), _ptr(b), dt, _ptr(h0),
              _ptr(out), _ptr(h_out), _ptr(sa), _ptr(ck), B, T, H, _stream(r))
    return out, h_out, sa, ck


class _WKV7Train(torch.autograd.Function):
    """Forward: checkpointing kernel.  Backward: checkpoint kernel v2, column-owned
    with recomputed states (or v1, the row-owned kernel that recovers them by
    dividing by w, WKV7Train.swift:99-205), the VJP of wkv7TrainWithState
    (WKV7Train.swift:410-467).  Gradients come
    back in each primal's dtype; the state gradient in the state's dtype."""

    @staticmethod
    def forward(ctx, r, w, k, v, a, b, h0):
        primals = [r, w, k, v, a, b]
        ins, dt = _prep(primals)
        B, T, H, D = ins[0].shape
        h = _state(h0, (B, H, D, D), ins[0].device)
        out, h_out, sa, ck = _train_forward(ins, dt, h)
        ctx.dt = dt
        ctx.dtypes = [x.dtype for x in primals]
        ctx.h0_dtype = None if h0 is None else h0.dtype
        ctx.keep = wkv7_keep_forward_outputs
        if ctx.keep:
            ctx.save_for_backward(*ins, h, sa, ck)
        else:
            ctx.save_for_backward(*ins, h)
        return out, h_out

    @staticmethod
    def backward(ctx, d_out, d_h_out):
        saved = ctx.saved_tensors
        ins = list(saved[:6])
        h = saved[6]
        if ctx.keep:
            sa, ck = saved[7], saved[8]
        else:   # recompute (gradient checkpointing of the kernel's own outputs)
            _, _, sa, ck = _train_forward(ins, ctx.dt, h)
        r = ins[0]
        B, T, H, D = r.shape
        dev = r.device
        d_out = (torch.zeros((B, T, H, D), dtype=torch.float32, device=dev) if d_out is None
                 else _aligned(d_out.to(torch.float32)))
        dho = None if d_h_out is None else _aligned(d_h_out.to(torch.float32))
        shared = len(set(ctx.dtypes)) == 1 and ctx.dtypes[0] in _DT
        gdt = ctx.dtypes[0] if shared else torch.float32
        grads = [torch.empty((B, T, H, D), dtype=gdt, device=dev) for _ in range(6)]
        dh_in = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
        variant = 2 if wkv7_backward_v2 else 1
        _lib.call("rwkv_wkv7_train_bwd", *[_ptr(x) for x in ins], ctx.dt, _ptr(h), _ptr(ck), _ptr(sa), _ptr(d_out),
                  _ptr(dho), *[_ptr(g) for g in grads], _DT[gdt], _ptr(dh_in), B, T, H, variant, _stream(r))
        grads = [g.to(t) for g, t in zip(grads, ctx.dtypes)]
        dh = None if ctx.h0_dtype is None else dh_in.to(ctx.h0_dtype)
        return (*grads, dh)


def wkv7_train_with_state(r, w, k, v, a, b, h_in=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Differentiable WKV-7 over T % 16 == 0 tokens with an explicit boundary
    state (WKV7Train.swift:375-468).  Returns (out, h_out); gradients flow to
    r..b and h_in."""
    B, T, H, D = r.shape
    if T % WKV7_CHUNK != 0:
        raise ValueError(f"T ({T}) must be a multiple of CHUNK {WKV7_CHUNK}")
    if D != WKV7_HEAD_SIZE:
        raise ValueError(f"D ({D}) must equal HEAD_SIZE {WKV7_HEAD_SIZE}")
    return _WKV7Train.apply(r, w, k, v, a, b, h_in)


def wkv7_train(r, w, k, v, a, b) -> torch.Tensor:
    """Zero initial state, final state dropped (WKV7Train.swift:472-475)."""
    return wkv7_train_with_state(r, w, k, v, a, b, None)[0]


def wkv7_train_forward_launches() -> int:
    return _lib.counters()["train_fwd"]


# ───────────────────────────── decode ─────────────────────────────

def wkv7_step_forward(r, w, k, v, a, b, h) -> Tuple[torch.Tensor, torch.Tensor]:
    """One token (WKV7DecodeKernels.swift:73-89).  r..b [H,S] (or [B,H,S] for
    B rows), h [H,S,S] (or [B,H,S,S]).  Returns (out, h') in fp32."""
    (r, w, k, v, a, b), dt = _prep([r, w, k, v, a, b], ndim_ok=(2, 3))
    squeeze = r.dim() == 2
    if squeeze:
        r, w, k, v, a, b = (x.unsqueeze(0) for x in (r, w, k, v, a, b))
    B, H, S = r.shape
    if S != WKV7_HEAD_SIZE:
        raise ValueError(f"S ({S}) must equal HEAD_SIZE {WKV7_HEAD_SIZE}")
    hs = (H, S, S) if squeeze else (B, H, S, S)
    if tuple(h.shape) != hs:
        raise ValueError(f"state {tuple(h.shape)}, expected {list(hs)}")
    h = _aligned(h.to(device=r.device, dtype=torch.float32))
    out = torch.empty((B, H, S), dtype=torch.float32, device=r.device)
    h_new = torch.empty((B, H, S, S), dtype=torch.float32, device=r.device)
    _lib.call("rwkv_wkv7_step", _ptr(r), _ptr(w), _ptr(k), _ptr(v), _ptr(a), _ptr(b), dt, _ptr(h), _ptr(out),
              _ptr(h_new), B, H, _stream(r))
    if squeeze:
        return out[0], h_new[0]
    return out, h_new


def _check_inplace(t: torch.Tensor, shape, device, what: str) -> None:
    """A caller buffer the kernel writes: fp32, contiguous, 16-byte aligned,
    of exactly `shape`, on the inputs' device."""
    if (t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != tuple(shape) or t.data_ptr() % 16
            or t.device != device):
        raise ValueError(f"{what} must be a contiguous, 16-byte aligned fp32 tensor of shape {list(shape)} on "
                         f"{device}, got {tuple(t.shape)} {t.dtype} on {t.device}")


def wkv7_step_(r, w, k, v, a, b, h, out=None) -> torch.Tensor:
    """In-place decode step for B rows: h [B,H,S,S] fp32 is updated in place
    (the C ABI allows h_in == h_out).  Returns out [B,H,S]."""
    (r, w, k, v, a, b), dt = _prep([r, w, k, v, a, b], ndim_ok=(3,))
    B, H, S = r.shape
    if S != WKV7_HEAD_SIZE:
        raise ValueError(f"S ({S}) must equal HEAD_SIZE {WKV7_HEAD_SIZE}")
    _check_inplace(h, (B, H, S, S), r.device, "in-place state")
    if out is None:
        out = torch.empty((B, H, S), dtype=torch.float32, device=r.device)
    else:
        _check_inplace(out, (B, H, S), r.device, "out")
    _lib.call("rwkv_wkv7_step", _ptr(r), _ptr(w), _ptr(k), _ptr(v), _ptr(a), _ptr(b), dt, _ptr(h), _ptr(out),
              _ptr(h), B, H, _stream(r))
    return out


def _pad_to_chunk(xs, T):
    """Pad the time axis with neutral steps (w = 1, others 0)."""
    Tp = -(-T // WKV7_CHUNK) * WKV7_CHUNK
    if Tp == T:
        return xs
    padded = []
    for idx, x in enumerate(xs):
        B, _, H, D = x.shape
        fill = 1.0 if idx == 1 else 0.0
        padded.append(torch.cat([x, torch.full((B, Tp - T, H, D), fill, dtype=x.dtype, device=x.device)], dim=1))
    return padded


def wkv7_steps(r, w, k, v, a, b, h_in=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Several tokens [B,T,H,D] (WKV7Step.swift:79-100).  Differentiable: when a
    gradient is needed the time axis is padded with neutral steps to the
    training kernel's CHUNK granularity (padding changes neither the state
    nor the gradients of the real steps)."""
    if r.dim() != 4:
        raise ValueError(f"wkv7_steps expects [B,T,H,D], got {tuple(r.shape)}")
    needs_grad = torch.is_grad_enabled() and any(
        x is not None and x.requires_grad for x in (r, w, k, v, a, b, h_in))
    if not needs_grad:
        return wkv7_sequence_forward(r, w, k, v, a, b, h_in)
    T = r.shape[1]
    xs = _pad_to_chunk([r, w, k, v, a, b], T)
    out, h = wkv7_train_with_state(*xs, h_in)
    return out[:, :T], h


def wkv7_step(r, w, k, v, a, b, h_in=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Exactly one token (WKV7Step.swift:45-67): [B,H,D] or [B,1,H,D] in,
    output of the same rank, state [B,H,D,D]."""
    if r.dim() == 4:
        if r.shape[1] != 1:
            raise ValueError(f"wkv7_step is exactly one token; use wkv7_steps for T={r.shape[1]}")
        return wkv7_steps(r, w, k, v, a, b, h_in)
    if r.dim() != 3:
        raise ValueError(f"wkv7_step expects [B,H,D] or [B,1,H,D], got {tuple(r.shape)}")
    out, h = wkv7_steps(*(x.unsqueeze(1) for x in (r, w, k, v, a, b)), h_in)
    return out[:, 0], h


def wkv_tail_applies(head_size: int) -> bool:
    """WKV7DecodeKernels.swift:92."""
    return bool(_lib.lib().rwkv_wkv_tail_applies(head_size))


def wkv_tail(wkv, r, k, v, r_k, ln_weight, ln_bias, gate, n_head: int, head_size: int, rows: int = 1,
             eps: float = 64e-5) -> torch.Tensor:
    """tmix tail for `rows` rows (WKV7DecodeKernels.swift:106-178): returns
    [rows, n_head·head_size] fp32."""
    if not wkv_tail_applies(head_size):
        raise ValueError(f"tail: S={head_size} is not a multiple of the SIMD width 32")
    Dm = n_head * head_size
    dev = wkv.device

    def rows_(x):
        return _aligned(x.reshape(rows, Dm).to(device=dev, dtype=torch.float32))

    def vec(x):
        return _aligned(x.reshape(Dm).to(device=dev, dtype=torch.float32))

    wkv_, r_, k_, v_, g_ = (rows_(x) for x in (wkv, r, k, v, gate))
    rk_, lw_, lb_ = (vec(x) for x in (r_k, ln_weight, ln_bias))
    out = torch.empty((rows, Dm), dtype=torch.float32, device=dev)
    _lib.call("rwkv_wkv_tail", _ptr(wkv_), _ptr(r_), _ptr(k_), _ptr(v_), _ptr(rk_), _ptr(lw_), _ptr(lb_), _ptr(g_),
              _ptr(out), rows, n_head, head_size, float(eps), _stream(wkv_))
    return out


def wkv7_step_tail_(r, w, k, v, a, b, h, r_k, ln_weight, ln_bias, gate, eps: float = 64e-5,
                    wkv_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Decode step followed by the tmix tail in one launch, fp32: h [B,H,S,S]
    is updated in place exactly as by wkv7_step_, and the result equals
    wkv_tail(wkv7_step_(...), r, k, v, ...) bitwise.  The pair
    wkv7StepForward + wkvTail of the reference's tmix decode step
    (WKV7DecodeKernels.swift:73-89, 106-178).  r..b, gate [B,H,S]; r_k,
    ln_weight, ln_bias [H·S].  `wkv_out` [B,H,S], when given, receives the step
    output.  Returns [B, H·S]."""
    xs = [r, w, k, v, a, b, gate]
    if any(x.dim() != 3 for x in xs):
        raise ValueError("step+tail: r, w, k, v, a, b and gate must be [B,H,S]")
    B, H, S = r.shape
    if S != WKV7_HEAD_SIZE or any(tuple(x.shape) != (B, H, S) for x in xs):
        raise ValueError(f"step+tail: inputs must share shape [B,H,{WKV7_HEAD_SIZE}]")
    dev = r.device
    if dev.type != "cuda":
        raise ValueError(f"step+tail inputs must live on a ROCm device, got {dev}")
    _check_inplace(h, (B, H, S, S), dev, "in-place state")
    r_, w_, k_, v_, a_, b_, g_ = (_aligned(x.to(device=dev, dtype=torch.float32)) for x in xs)
    rk_, lw_, lb_ = (_aligned(x.reshape(H * S).to(device=dev, dtype=torch.float32)) for x in (r_k, ln_weight, ln_bias))
    if wkv_out is not None:
        _check_inplace(wkv_out, (B, H, S), dev, "wkv_out")
    out = torch.empty((B, H * S), dtype=torch.float32, device=dev)
    _lib.call("rwkv_wkv7_step_tail", _ptr(r_), _ptr(w_), _ptr(k_), _ptr(v_), _ptr(a_), _ptr(b_), _ptr(h), _ptr(h),
              _ptr(rk_), _ptr(lw_), _ptr(lb_), _ptr(g_), _ptr(wkv_out) if wkv_out is not None else None, _ptr(out),
              B, H, float(eps), _stream(r_))
    return out

