"""numpy front end of the C oracle (oracle/oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by
the cpu_baseline leg of bench.py, always as the reference results are
compared with (or the timed CPU restatement), never by the product package
swiftrwkv_amd/.

Each wrapper names the reference lines its C function restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
HEAD = 64
CHUNK = 16

_lib = None


def build() -> str:
    """Compile liboracle.so from oracle.c with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = ctypes.c_void_p
I = ctypes.c_int
L = ctypes.c_int64


def _declare(c):
    c.orc_f32_to_f16.restype = ctypes.c_uint16
    c.orc_f32_to_f16.argtypes = [ctypes.c_float]
    c.orc_f16_to_f32.restype = ctypes.c_float
    c.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    for name in ("orc_f32_to_f16_array", "orc_f16_to_f32_array", "orc_f32_to_bf16_array"):
        getattr(c, name).argtypes = [P, P, L]
        getattr(c, name).restype = None
    c.orc_wkv7_fwd_f32.argtypes = [P] * 11 + [I, I, I, I]
    c.orc_wkv7_fwd_f64.argtypes = [P] * 10 + [I, I, I]
    c.orc_wkv7_bwd_f64.argtypes = [P] * 16 + [I, I, I]
    c.orc_wkv_tail_f64.argtypes = [P] * 9 + [I, I, I, ctypes.c_double]
    c.orc_unpack6x8.argtypes = [P, L, P]
    c.orc_sb6_to_k3.argtypes = [P] * 6 + [L, L] + [P] * 3
    c.orc_sym_interleave.argtypes = [P, P, P, L, L, P]
    c.orc_sb6_dequant.argtypes = [P, P, P, L, L, I, P, I]
    c.orc_sym_dequant.argtypes = [P, P, P, L, L, I, P, I]
    c.orc_sb6_gemv_f64.argtypes = [P, I, P, P, P, L, L, I, P]
    c.orc_sym_gemv_f64.argtypes = [P, I, P, P, P, L, L, I, L, P]
    c.orc_cpu_sb6_dequant_matvec.argtypes = [P, P, P, P, L, L, I, P, I]
    c.orc_cpu_wkv7_step.argtypes = [P] * 8 + [I, I, I]
    c.orc_max_threads.restype = I
    for f in ("orc_wkv7_fwd_f32", "orc_wkv7_fwd_f64", "orc_wkv7_bwd_f64", "orc_wkv_tail_f64",
              "orc_unpack6x8", "orc_sb6_to_k3", "orc_sym_interleave", "orc_sb6_dequant",
              "orc_sym_dequant", "orc_sb6_gemv_f64", "orc_sym_gemv_f64",
              "orc_cpu_sb6_dequant_matvec", "orc_cpu_wkv7_step"):
        getattr(c, f).restype = None


def _p(a):
    return None if a is None else a.ctypes.data_as(P)


def _c(a, dt):
    return None if a is None else np.ascontiguousarray(a, dtype=dt)


# ───────────────────────────── conversions ─────────────────────────────

def f32_to_f16_bits(x) -> np.ndarray:
    """RNE float32 → binary16 bit patterns (uint16)."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def f32_to_bf16_bits(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_array(_p(x), _p(out), x.size)
    return out


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ───────────────────────────── WKV-7 ─────────────────────────────

def wkv7_fwd_f32(r, w, k, v, a, b, h_in=None, want_sa=False, want_ckpt=False, nthreads=0):
    """WKV7.swift:207-224 order in fp32.  Inputs [B,T,H,64]; returns
    (out, h_out[, sa][, ckpt])."""
    r, w, k, v, a, b = (_c(x, np.float32) for x in (r, w, k, v, a, b))
    B, T, H, Dh = r.shape
    assert Dh == HEAD
    h_in = _c(h_in, np.float32)
    out = np.empty_like(r)
    h_out = np.empty((B, H, HEAD, HEAD), np.float32)
    sa = np.empty_like(r) if want_sa else None
    ck = np.empty((B, H, T // CHUNK, HEAD, HEAD), np.float32) if want_ckpt else None
    lib().orc_wkv7_fwd_f32(_p(r), _p(w), _p(k), _p(v), _p(a), _p(b), _p(h_in), _p(out), _p(h_out),
                           _p(sa), _p(ck), B, T, H, nthreads)
    res = [out, h_out]
    if want_sa:
        res.append(sa)
    if want_ckpt:
        res.append(ck)
    return tuple(res)


def wkv7_fwd_f64(r, w, k, v, a, b, h_in=None, want_sa=False):
    r, w, k, v, a, b = (_c(x, np.float64) for x in (r, w, k, v, a, b))
    B, T, H, Dh = r.shape
    assert Dh == HEAD
    h_in = _c(h_in, np.float64)
    out = np.empty_like(r)
    h_out = np.empty((B, H, HEAD, HEAD), np.float64)
    sa = np.empty_like(r) if want_sa else None
    lib().orc_wkv7_fwd_f64(_p(r), _p(w), _p(k), _p(v), _p(a), _p(b), _p(h_in), _p(out), _p(h_out),
                           _p(sa), B, T, H)
    return (out, h_out, sa) if want_sa else (out, h_out)


def wkv7_bwd_f64(r, w, k, v, a, b, h_in, d_out, d_h_out=None):
    """Analytic reverse pass (WKV7Train.swift:276-325 equations) with stored
    fp64 states.  Returns (dr, dw, dk, dv, da, db, dh_in)."""
    r, w, k, v, a, b, d_out = (_c(x, np.float64) for x in (r, w, k, v, a, b, d_out))
    B, T, H, _ = r.shape
    h_in = _c(h_in, np.float64)
    d_h_out = _c(d_h_out, np.float64)
    g = [np.empty_like(r) for _ in range(6)]
    dh_in = np.empty((B, H, HEAD, HEAD), np.float64)
    lib().orc_wkv7_bwd_f64(_p(r), _p(w), _p(k), _p(v), _p(a), _p(b), _p(h_in), _p(d_out), _p(d_h_out),
                           *[_p(x) for x in g], _p(dh_in), B, T, H)
    return (*g, dh_in)


def wkv_tail_f64(wkv, r, k, v, rk, lnw, lnb, g, N, H, S, eps=64e-5):
    """WKV7DecodeKernels.swift:124-156 in fp64; returns [N, H*S]."""
    arrs = [_c(x, np.float32).reshape(-1) for x in (wkv, r, k, v, rk, lnw, lnb, g)]
    out = np.empty(N * H * S, np.float64)
    lib().orc_wkv_tail_f64(*[_p(x) for x in arrs], _p(out), N, H, S, eps)
    return out.reshape(N, H * S)


# ───────────────────────────── .rwkvq ─────────────────────────────

def unpack6x8(b) -> np.ndarray:
    """RwkvqFile.swift:171-181: uint8 [..., 6] → int32 [..., 8]."""
    b = _c(b, np.uint8)
    assert b.shape[-1] == 6
    n = b.size // 6
    out = np.empty(b.shape[:-1] + (8,), np.int32)
    lib().orc_unpack6x8(_p(b), n, _p(out))
    return out


def sb6_to_k3(codes_packed, qh, qh2, gw_qsqm, gw_d, gw_dm, OUT, IN):
    """RwkvqFile.swift:189-212.  gw_d / gw_dm as uint16 fp16 bit patterns."""
    NB = IN // 32
    xbits = (qh is not None) + (qh2 is not None)
    cp = _c(codes_packed, np.uint8)
    qh = _c(qh, np.uint8)
    qh2 = _c(qh2, np.uint8)
    qsqm_d = _c(gw_qsqm, np.uint8)
    d = _c(gw_d, np.uint16)
    dm = _c(gw_dm, np.uint16)
    qblk = np.empty((OUT, NB * (16 + 4 * xbits)), np.uint8)
    qsqm = np.empty((OUT, NB * 2), np.uint8)
    ddm = np.empty((OUT, (NB // 8) * 2), np.uint16)
    lib().orc_sb6_to_k3(_p(cp), _p(qh), _p(qh2), _p(qsqm_d), _p(d), _p(dm), OUT, IN, _p(qblk), _p(qsqm), _p(ddm))
    return qblk, qsqm, ddm, xbits


def sym_interleave(codes_packed, qh, qh2, OUT, IN):
    """RwkvqFile.swift:437-449."""
    qblk = np.empty((OUT, IN // 32 * 24), np.uint8)
    lib().orc_sym_interleave(_p(_c(codes_packed, np.uint8)), _p(_c(qh, np.uint8)), _p(_c(qh2, np.uint8)),
                             OUT, IN, _p(qblk))
    return qblk


_DT = {"f32": (0, np.float32), "bf16": (1, np.uint16), "f16": (2, np.uint16)}


def sb6_dequant(qblk, qsqm, ddm, OUT, IN, xbits, out_dt="f32"):
    """RwkvqDequant.swift:116-140; bf16/f16 results returned as uint16 bits."""
    code, npdt = _DT[out_dt]
    out = np.empty((OUT, IN), npdt)
    lib().orc_sb6_dequant(_p(_c(qblk, np.uint8)), _p(_c(qsqm, np.uint8)), _p(_c(ddm, np.uint16)),
                          OUT, IN, xbits, _p(out), code)
    return out


def sym_dequant(qblk, qs, d, OUT, IN, bits, out_dt="f32"):
    """RwkvqDequant.swift:350-388 / :442-466."""
    code, npdt = _DT[out_dt]
    out = np.empty((OUT, IN), npdt)
    lib().orc_sym_dequant(_p(_c(qblk, np.uint8)), _p(_c(qs, np.uint8)), _p(_c(d, np.uint16)),
                          OUT, IN, bits, _p(out), code)
    return out


def sb6_gemv_f64(x, qblk, qsqm, ddm, OUT, IN, xbits):
    """fp64 anchor of RwkvqSb6GEMV.swift:118-144 over N rows of x."""
    x = _c(x, np.float32).reshape(-1, IN)
    N = x.shape[0]
    y = np.empty((N, OUT), np.float64)
    lib().orc_sb6_gemv_f64(_p(x), N, _p(_c(qblk, np.uint8)), _p(_c(qsqm, np.uint8)), _p(_c(ddm, np.uint16)),
                           OUT, IN, xbits, _p(y))
    return y


def sym_gemv_f64(x, qblk, qs, d, OUT, IN, bits, out_per=None):
    """fp64 anchor of RwkvqSymGEMV.swift:126-199 (x row n·NK + row/out_per)."""
    out_per = OUT if out_per is None else out_per
    x = _c(x, np.float32).reshape(-1, IN)
    NK = OUT // out_per
    N = x.shape[0] // NK
    y = np.empty((N, OUT), np.float64)
    lib().orc_sym_gemv_f64(_p(x), N, _p(_c(qblk, np.uint8)), _p(_c(qs, np.uint8)), _p(_c(d, np.uint16)),
                           OUT, IN, bits, out_per, _p(y))
    return y


def sb6_matmul_f16_base(x, qblk, qsqm, ddm, OUT, IN, xbits=0):
    """The long pass of X070Backbone.baseMatmul with an fp16 base
    (X070Backbone.swift:337-356): W16 = the fp16 dequant (RwkvqDequant.swift:116-140
    stored as fp16), x rounded to fp16, and their product summed exactly
    (fp64: the fp16·fp16 products and their sums over these sizes are exact
    to 2^-52) — the value the fp16 matmul's output rounds.  Returns
    (exact [N, OUT], magnitude Σ|x16·w16| [N, OUT]); the magnitude scales the
    accumulation error an fp32 sum of the same products may carry."""
    W16 = sb6_dequant(qblk, qsqm, ddm, OUT, IN, xbits, "f16").view(np.float16).astype(np.float64)
    x16 = np.asarray(x, np.float32).reshape(-1, IN).astype(np.float16).astype(np.float64)
    return x16 @ W16.T, np.abs(x16) @ np.abs(W16).T


def sym_matmul_f16_base(x, qblk, qs, d, OUT, IN, bits):
    """sb6_matmul_f16_base for a sym matrix: W16 = the fp16 dequant of
    rwkvqDequantSym (RwkvqDequant.swift:350-388, its fp16 branch computing in
    half), x rounded to fp16, the product summed exactly.  Returns (exact
    [N, OUT], magnitude Σ|x16·w16| [N, OUT])."""
    W16 = sym_dequant(qblk, qs, d, OUT, IN, bits, "f16").view(np.float16).astype(np.float64)
    x16 = np.asarray(x, np.float32).reshape(-1, IN).astype(np.float16).astype(np.float64)
    return x16 @ W16.T, np.abs(x16) @ np.abs(W16).T


# ───────────────────────────── CPU baseline ─────────────────────────────

def cpu_sb6_dequant_matvec(x, qblk, qsqm, ddm, OUT, IN, xbits, nthreads):
    x = _c(x, np.float32)
    y = np.empty(OUT, np.float32)
    lib().orc_cpu_sb6_dequant_matvec(_p(x), _p(qblk), _p(qsqm), _p(ddm), OUT, IN, xbits, _p(y), nthreads)
    return y


def cpu_wkv7_step(r, w, k, v, a, b, h, out, B, H, nthreads):
    lib().orc_cpu_wkv7_step(_p(r), _p(w), _p(k), _p(v), _p(a), _p(b), _p(h), _p(out), B, H, nthreads)


def max_threads() -> int:
    return int(lib().orc_max_threads())
