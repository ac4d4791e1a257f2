"""ctypes binding of libswiftrwkv_hip.so (the C ABI in include/rwkv_hip.h).

The library is built in-tree by swiftrwkv_amd/build.py.  There is no fallback:
if the shared library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

# torch first: its bundled libamdhip64.so.7 / libhsa-runtime64.so.1 are then
# the ones our library binds to (same SONAME), so there is exactly one HIP
# runtime in the process and torch's streams and pointers are valid here.
import torch  # noqa: F401

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libswiftrwkv_hip.so")

P = ctypes.c_void_p
I = ctypes.c_int
L = ctypes.c_int64
F = ctypes.c_float

RWKV_OK = 0
STATUS_NAMES = {0: "ok", 1: "shape", 2: "dtype", 3: "unsupported", 4: "format", 5: "hip", 6: "null", 7: "io"}

F32, BF16, F16 = 0, 1, 2


class RwkvHipError(RuntimeError):
    """A non-OK rwkv_status from the C ABI."""

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"[{STATUS_NAMES.get(status, status)}] {message}")


class Counters(ctypes.Structure):
    _fields_ = [(n, L) for n in ("seq_fwd", "chunk_fwd", "train_fwd", "train_bwd", "step", "tail",
                                 "sb6_dequant", "sym_dequant", "sb6_gemv", "sym_gemv", "sym_fused",
                                 "step_tail", "sb6_fused", "sym_rows", "x070", "sb6_gemm", "seq_chunked",
                                 "sb6_batch", "sym_gemm")]


class Finding(ctypes.Structure):
    """rwkvq_finding: why a manifest was rejected."""
    _fields_ = [("kind", I), ("tensor", ctypes.c_char * 192), ("buffer", ctypes.c_char * 32),
                ("n_expected", I), ("n_got", I), ("expected", L * 4), ("got", L * 4)]


class TensorDesc(ctypes.Structure):
    """rwkvq_tensor: one validated manifest entry."""
    _fields_ = [("key", ctypes.c_char_p), ("kind", I), ("ndim", I), ("shape", L * 8), ("bits", I), ("xbits", I),
                ("group_size", I), ("super_block", I), ("transposed", I), ("packed", I), ("outliers", L)]


class ModelDesc(ctypes.Structure):
    """rwkvq_model: the manifest's model-level fields."""
    _fields_ = [("format_version", I), ("naming", ctypes.c_char_p), ("n_layer", L), ("n_embd", L),
                ("head_size", L), ("vocab_size", L)]


# name → (restype, argtypes)
_SIGS = {
    "rwkv_abi_version": (I, []),
    "rwkv_status_string": (ctypes.c_char_p, [I]),
    "rwkv_last_error": (ctypes.c_char_p, []),
    "rwkv_wkv7_head_size": (I, []),
    "rwkv_wkv7_chunk": (I, []),
    "rwkv_wkv7_seq_fwd": (I, [P] * 6 + [I, P, P, P, L, L, L, P]),
    "rwkv_wkv7_chunk_fwd": (I, [P] * 6 + [I, P, P, P, P, L, L, L, P]),
    "rwkv_wkv7_chunked_workspace": (L, [L, L, L]),
    "rwkv_sb6_gemv_batch_applies": (I, [L, L, L, I, L]),
    "rwkv_sb6_gemv_batch_workspace": (L, [L, L, L, L]),
    "rwkv_sb6_gemv_batch": (I, [P, L, P, P, P, P, L, L, I, L, I, P, L, P]),
    "rwkv_sb6_t16_pack": (I, [P, P, P, L, L, P, P, P, P]),
    "rwkv_sb6_gemv_batch_t16": (I, [P, L, P, P, P, P, L, L, L, I, P, L, P]),
    "rwkv_sb6_gemv_batch_t16_rows": (I, [P, L, P, P, P, P, L, L, L, I, P]),
    "rwkv_sb6_gemv_batch_t16_launches": (I, [L, L, L, L]),
    "rwkv_wkv7_seq_fwd_chunked": (I, [P] * 6 + [I, P, P, P, L, L, L, P, L, P]),
    "rwkv_wkv7_seq_fwd_chunked_static": (I, [P] * 6 + [I, P, P, P, L, L, L, P]),
    "rwkv_wkv7_train_fwd": (I, [P] * 6 + [I, P, P, P, P, P, L, L, L, P]),
    "rwkv_wkv7_train_bwd": (I, [P] * 6 + [I, P, P, P, P, P] + [P] * 6 + [I, P, L, L, L, I, P]),
    "rwkv_wkv7_step": (I, [P] * 6 + [I, P, P, P, L, L, P]),
    "rwkv_wkv7_step_tail": (I, [P] * 14 + [L, L, F, P]),
    "rwkv_wkv_tail_applies": (I, [L]),
    "rwkv_wkv_tail": (I, [P] * 9 + [L, L, L, F, P]),
    "rwkv_wkv_tail_to": (I, [P] * 9 + [I, L, L, L, F, P]),
    "rwkv_sb6_dequant": (I, [P, P, P, P, I, L, L, I, P]),
    "rwkv_sym_dequant": (I, [P, P, P, P, I, L, L, I, P]),
    "rwkv_sym_rows": (I, [P, L, P, P, P, P, I, L, L, I, P]),
    "rwkv_sb6_gemv_applies": (I, [L, L, I, I, L]),
    "rwkv_sb6_gemv": (I, [P, L, P, P, P, P, L, L, I, P]),
    "rwkv_sb6_gemv_fused": (I, [P, L, P, P, P, P, L, L, I, L, P]),
    "rwkv_sym_gemv_applies": (I, [L, L, I, L]),
    "rwkv_sym_gemv": (I, [P, L, P, P, P, P, L, L, I, L, P]),
    "rwkv_sb6_gemv_ep": (I, [P, L, P, P, P, P, L, L, I, I, P]),
    "rwkv_sym_gemv_ep": (I, [P, L, P, P, P, P, L, L, I, I, P]),
    "rwkv_sb6_gemm_applies": (I, [L, L, I, L]),
    "rwkv_sb6_gemm": (I, [P, I, L, L, L, P, P, P, P, L, L, L, I, L, I, P, L, P]),
    "rwkv_quant_gemm_workspace": (L, [L, L, L]),
    "rwkv_f16_gemm_applies": (I, [L, L, L, L]),
    "rwkv_f16_gemm": (I, [P, L, L, L, P, P, L, L, L, L, I, P]),
    "rwkv_sym_gemm_applies": (I, [L, L, I, L]),
    "rwkv_x070_seq_lora": (I, [P, L, L, P, P, P, P, P, I, L, L, L, L, I, P, P, P, P, P, P]),
    "rwkv_x070_seq_lora_split": (I, [L, L, I, L, L, L, L]),
    "rwkv_sym_gemm": (I, [P, I, L, L, L, P, P, P, P, L, L, L, I, L, I, P, L, P]),
    "rwkv_layer_norm": (I, [P, I, P, L, P, P, P, L, L, F, P]),
    "rwkv_x070_seq_shift_mix": (I, [P, P, P, P, P, I, I, P, I, L, L, P, L, L, I, L, L, L, P]),
    "rwkv_x070_seq_tmix_pre": (I, [P] * 10 + [I, P] + [P] * 7 + [L, L, L, P]),
    "rwkv_x070_shift_mix": (I, [P, P, P, P, P, I, P, P, L, L, F, P]),
    "rwkv_x070_lora_in": (I, [P, P, I, L, L, L, L, I, P, L, L, P]),
    "rwkv_x070_rkv_lora": (I, [P, P, P, P, P, L, L, I, L, P, P, I, L, L, L, L, I, P, P]),
    "rwkv_x070_tmix_core": (I, [P, P, P, P, P, P, I, L, L, L, L] + [P] * 8 + [P, I, P, P, L, L, F, P, P, P]),
    "rwkv_x070_ln_fused_applies": (I, [L, L, I]),
    "rwkv_x070_rkv_lora_ln": (I, [P] * 5 + [F, P, P, P, P, P, L, I, P, I, L, L, L, L, I, P, P]),
    "rwkv_x070_ffn_key_ln": (I, [P] * 5 + [F, P, P, P, P, P, L, L, I, P]),
    "rwkv_x070_ffn_value": (I, [P, P, P, P, P, L, L, I, P, P, P]),
    "rwkv_unpack6x8": (I, [P, L, P]),
    "rwkv_sb6_to_k3": (I, [P] * 6 + [L, L, P, P, P]),
    "rwkv_sym_interleave": (I, [P, P, P, L, L, P]),
    "rwkvq_encode_sb6": (I, [P, L, L, I, P, P, P, P, P, P, I]),
    "rwkvq_encode_sym": (I, [P, L, L, I, P, P, P, P, P, P, I]),
    "rwkvq_open": (I, [ctypes.c_char_p, ctypes.POINTER(P)]),
    "rwkvq_close": (None, [P]),
    "rwkvq_count": (L, [P]),
    "rwkvq_entry": (I, [P, L, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_char_p),
                        ctypes.POINTER(I), ctypes.POINTER(ctypes.POINTER(L)), ctypes.POINTER(P),
                        ctypes.POINTER(L)]),
    "rwkvq_metadata": (ctypes.c_char_p, [P, ctypes.c_char_p]),
    "rwkvq_manifest_read": (I, [P, I, ctypes.POINTER(P), ctypes.POINTER(Finding)]),
    "rwkvq_manifest_free": (None, [P]),
    "rwkvq_manifest_count": (L, [P]),
    "rwkvq_manifest_tensor": (I, [P, L, ctypes.POINTER(TensorDesc)]),
    "rwkvq_manifest_model": (I, [P, ctypes.POINTER(ModelDesc)]),
    "rwkvq_read_sb6": (I, [P, P, L, P, P, P]),
    "rwkvq_read_sym": (I, [P, P, L, P, P, P]),
    "rwkv_time_next_launch": (I, [P, P]),
    "rwkv_get_counters": (None, [ctypes.POINTER(Counters)]),
    "rwkv_reset_counters": (None, []),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load the in-tree HIP library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m swiftrwkv_amd.build` "
                "(there is no CPU fallback for the HIP path)")
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def exported_symbols():
    return list(_SIGS)


def check(status: int) -> None:
    if status != RWKV_OK:
        msg = lib().rwkv_last_error()
        raise RwkvHipError(status, msg.decode() if msg else "")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


def counters() -> dict:
    c = Counters()
    lib().rwkv_get_counters(ctypes.byref(c))
    return {n: getattr(c, n) for n, _ in Counters._fields_}


def reset_counters() -> None:
    lib().rwkv_reset_counters()
