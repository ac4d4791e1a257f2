"""RWKVQuant on MI355X: the Swift module's public API over the HIP C ABI.

Mirrors Sources/RWKVQuant/*.swift: the .rwkvq safetensors container
(RwkvqFile.swift), the manifest / sidecar object with `dequantize`
(RwkvqSidecar.swift), the fused dequant kernels (RwkvqDequant.swift) and the
decode GEMVs with r/k/v fusion (RwkvqSb6GEMV.swift, RwkvqSymGEMV.swift).
Dequant and GEMV run in libswiftrwkv_hip.so; container parsing, the K3 /
sym interleave repack and the encoders run in its host C++ part.

Also here (not in the reference, which only decodes files produced by the
external rwkv-quant project): `encode_sb6` / `encode_sym` and `write_rwkvq`,
used to produce seeded synthetic .rwkvq files.
"""
from __future__ import annotations

import ctypes
import enum
import json
import os
from dataclasses import dataclass
from typing import Callable, Dict, Iterable, List, Optional, Tuple

import numpy as np
import torch

from . import _lib

# ───────────────────────────── errors / kinds ─────────────────────────────


class RwkvqError(Exception):
    """RwkvqError (RwkvqSidecar.swift:25-56)."""


class MissingFile(RwkvqError):
    pass


class MalformedManifest(RwkvqError):
    pass


class MissingBuffer(RwkvqError):
    def __init__(self, tensor: str, buffer: str):
        self.tensor, self.buffer = tensor, buffer
        super().__init__(f"no buffer {buffer} for tensor {tensor}")


class ShapeMismatch(RwkvqError):
    def __init__(self, tensor: str, expected, got):
        self.tensor, self.expected, self.got = tensor, list(expected), list(got)
        super().__init__(f"{tensor}: expected shape {self.expected}, file has {self.got}")


class UnsupportedKind(RwkvqError):
    def __init__(self, tensor: str, kind: str):
        self.tensor, self.kind = tensor, kind
        super().__init__(f"{tensor}: {kind}")


class PartialExport(RwkvqError):
    """RwkvqError.partialExport: the file holds only compressed projections,
    no dense model body (X070Backbone load(fromSidecar:))."""

    def __init__(self, tensors: int):
        self.tensors = tensors
        super().__init__(f"partial export: {tensors} tensors, none of them dense")


class IncompleteManifest(RwkvqError):
    """RwkvqFullConvertError.incompleteManifest (RwkvqFullConvert.swift:31-39)."""


class RwkvqKind(str, enum.Enum):
    """RwkvqKind (RwkvqSidecar.swift:60-67)."""
    sb6 = "sb6"
    sym = "sym"
    asym = "asym"
    rtn = "rtn"
    dense = "dense"


@dataclass(frozen=True)
class RwkvqTensorInfo:
    """RwkvqTensorInfo (RwkvqSidecar.swift:75-99)."""
    kind: RwkvqKind
    shape: Tuple[int, ...]
    bits: int
    xbits: int
    group_size: int
    super_block: int
    packed: bool
    outlier_count: int
    transposed: bool

    @property
    def is_sb6(self) -> bool:
        return self.kind == RwkvqKind.sb6

    @property
    def is_quantized_base(self) -> bool:
        return self.kind in (RwkvqKind.sb6, RwkvqKind.sym)

    @property
    def out_features(self) -> int:
        return self.shape[0]

    @property
    def in_features(self) -> int:
        return self.shape[1]


def is_raw_lora_world(key: str) -> bool:
    """RwkvqNaming.isRawLoRAWorld: world checkpoints keep att.{w,a,v,g}{1,2}
    as [in, out] (RwkvqFileTests.swift:123-127)."""
    parts = key.split(".")
    return (len(parts) == 4 and parts[0] == "blocks" and parts[2] == "att" and len(parts[3]) == 2
            and parts[3][0] in "wavg" and parts[3][1] in "12")


# ───────────────────────────── container ─────────────────────────────

_ST_NP = {"BOOL": np.bool_, "U8": np.uint8, "I8": np.int8, "I16": np.int16, "U16": np.uint16,
          "F16": np.float16, "BF16": np.uint16, "I32": np.int32, "U32": np.uint32, "F32": np.float32,
          "F64": np.float64, "I64": np.int64, "U64": np.uint64}


class RwkvqContainer:
    """Memory-mapped safetensors container (RwkvqFile.swift:31-162), parsed
    and validated by the C ABI (rwkvq_open)."""

    def __init__(self, path: str):
        p = os.path.expanduser(path)
        h = ctypes.c_void_p()
        st = _lib.lib().rwkvq_open(p.encode(), ctypes.byref(h))
        if st != _lib.RWKV_OK:
            msg = _lib.lib().rwkv_last_error().decode()
            if st == 7:
                raise MissingFile(msg)
            raise MalformedManifest(msg)
        self._h = h
        self._entries: Dict[str, tuple] = {}
        name, dt, nd = ctypes.c_char_p(), ctypes.c_char_p(), ctypes.c_int()
        shp, data, nb = ctypes.POINTER(ctypes.c_int64)(), ctypes.c_void_p(), ctypes.c_int64()
        for i in range(_lib.lib().rwkvq_count(h)):
            _lib.check(_lib.lib().rwkvq_entry(h, i, ctypes.byref(name), ctypes.byref(dt), ctypes.byref(nd),
                                              ctypes.byref(shp), ctypes.byref(data), ctypes.byref(nb)))
            shape = tuple(shp[j] for j in range(nd.value))
            self._entries[name.value.decode()] = (dt.value.decode(), shape, data.value, nb.value)
        self.metadata: Dict[str, str] = {}
        for key in ("rwkvq", "format"):
            v = _lib.lib().rwkvq_metadata(h, key.encode())
            if v is not None:
                self.metadata[key] = v.decode()

    def close(self):
        if getattr(self, "_h", None):
            _lib.lib().rwkvq_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def names(self) -> List[str]:
        return sorted(self._entries)

    def contains(self, name: str) -> bool:
        return name in self._entries

    def shape(self, name: str) -> Optional[Tuple[int, ...]]:
        e = self._entries.get(name)
        return None if e is None else e[1]

    def dtype(self, name: str) -> Optional[str]:
        e = self._entries.get(name)
        return None if e is None else e[0]

    def array(self, name: str, as_dtype=None) -> Optional[np.ndarray]:
        """Copy of one buffer (numpy).  `as_dtype` reinterprets the bytes as
        another type of the same size (RwkvqFile.swift:154-161)."""
        e = self._entries.get(name)
        if e is None:
            return None
        dt, shape, ptr, nbytes = e
        npdt = np.dtype(_ST_NP[dt])
        if as_dtype is not None:
            if np.dtype(as_dtype).itemsize != npdt.itemsize:
                raise ValueError(f"{name}: {dt} cannot be read as {as_dtype} (element size differs)")
            npdt = np.dtype(as_dtype)
        if nbytes == 0:
            return np.zeros(shape, npdt)
        raw = (ctypes.c_uint8 * nbytes).from_address(ptr)
        return np.frombuffer(raw, dtype=np.uint8).copy().view(npdt).reshape(shape)


# ───────────────────────────── host repack ─────────────────────────────

def _np_ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def rwkvq_unpack6x8(b: np.ndarray) -> np.ndarray:
    """RwkvqFile.swift:171-181: uint8 [..., 6] → int32 [..., 8]."""
    b = np.ascontiguousarray(b, dtype=np.uint8)
    if b.shape[-1] != 6:
        raise ValueError(f"unpack6: expected 6 bytes per super-block, not {b.shape[-1]}")
    out = np.empty(b.shape[:-1] + (8,), np.int32)
    _lib.call("rwkv_unpack6x8", _np_ptr(b), b.size // 6, _np_ptr(out))
    return out


def rwkvq_sb6_to_k3(codes_packed, qsqm, d, dm, qh, qh2, shape, group_size=32, super_block=8):
    """RwkvqFile.swift:189-212 → (qblk, qsqm, ddm, xbits) as numpy arrays."""
    OUT, IN = shape
    if group_size != 32 or super_block != 8:
        raise ValueError("sb6 K3 repack is defined for block 32, super-block 8")
    NB = IN // 32
    xbits = (qh is not None) + (qh2 is not None)

    def bits16(x):   # fp16 scales travel as their bit patterns
        x = np.ascontiguousarray(x)
        if x.dtype == np.float16:
            return x.view(np.uint16)
        if x.dtype != np.uint16:
            raise ValueError(f"sb6 scales must be fp16 (or their uint16 bits), got {x.dtype}")
        return x

    c = [np.ascontiguousarray(x, dtype=np.uint8) if x is not None else None
         for x in (codes_packed, qh, qh2, qsqm)] + [bits16(d), bits16(dm)]
    qblk = np.empty((OUT, NB * (16 + 4 * xbits)), np.uint8)
    k3 = np.empty((OUT, NB * 2), np.uint8)
    ddm = np.empty((OUT, (NB // 8) * 2), np.uint16)
    _lib.call("rwkv_sb6_to_k3", *[_np_ptr(x) for x in c], OUT, IN, _np_ptr(qblk), _np_ptr(k3), _np_ptr(ddm))
    return qblk, k3, ddm, xbits


def rwkvq_sym_interleave(codes_packed, qh, qh2, shape) -> np.ndarray:
    """RwkvqFile.swift:437-449: sym 6-bit → [OUT, IN/32·24]."""
    OUT, IN = shape
    qblk = np.empty((OUT, IN // 32 * 24), np.uint8)
    c = [np.ascontiguousarray(x, dtype=np.uint8) for x in (codes_packed, qh, qh2)]
    _lib.call("rwkv_sym_interleave", *[_np_ptr(x) for x in c], OUT, IN, _np_ptr(qblk))
    return qblk


# ───────────────────────────── kernels (dequant / GEMV) ─────────────────────────────

_OUT_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous with a 16-byte aligned base (the kernels use vector loads)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _dev_u8(t: torch.Tensor, numel: int, what: str) -> torch.Tensor:
    if t.device.type != "cuda":
        raise ValueError("quantised buffers must live on a ROCm device for the HIP kernels")
    if t.dtype not in (torch.uint8, torch.int8):
        raise ValueError(f"{what}: expected a byte buffer, got {t.dtype}")
    if t.numel() != numel:
        raise ValueError(f"{what}: {t.numel()} bytes, the shape needs {numel}")
    return _aligned(t)


def _dev_f16(t: torch.Tensor, numel: int, what: str) -> torch.Tensor:
    if t.dtype != torch.float16:
        raise ValueError(f"{what}: expected fp16 scales, got {t.dtype}")
    if t.numel() != numel:
        raise ValueError(f"{what}: {t.numel()} scales, the shape needs {numel}")
    return _aligned(t)


def _sb6_bufs(qblk, qsqm, ddm, OUT, IN, xbits):
    if IN % 256 or xbits not in (0, 1, 2):
        raise ValueError(f"sb6: IN={IN} must be a multiple of 256 and xbits in 0...2")
    NB = IN // 32
    return (_dev_u8(qblk, OUT * NB * (16 + 4 * xbits), "qblk"), _dev_u8(qsqm, OUT * NB * 2, "qsqm"),
            _dev_f16(ddm, OUT * (NB // 8) * 2, "ddm"))


def _sym_bufs(qblk, qs, d, OUT, IN, bits):
    if bits not in (6, 8) or IN % (16 if bits == 8 else 32):
        raise ValueError(f"sym: bits={bits}, IN={IN} not taken")
    NB = IN // 16
    return (_dev_u8(qblk, OUT * (IN if bits == 8 else IN // 32 * 24), "qblk"), _dev_u8(qs, OUT * NB, "qs"),
            _dev_f16(d, OUT * ((NB + 15) // 16), "d"))


def rwkvq_dequant_dense(qblk, qsqm, ddm, out_features: int, in_features: int, super_block: int, xbits: int,
                        dtype=torch.float32) -> torch.Tensor:
    """packed sb6 → dense [OUT, IN] in one launch (RwkvqDequant.swift:160-183).
    Combine always in fp32; `dtype` is only the storage type."""
    if super_block != 8:
        raise ValueError(f"sb6 dequant: super-block {super_block}, the kernel is built for 8")
    if dtype not in _OUT_DT:
        raise ValueError(f"dequant to {dtype} is not supported")
    qblk, qsqm, ddm = _sb6_bufs(qblk, qsqm, ddm, out_features, in_features, xbits)
    out = torch.empty((out_features, in_features), dtype=dtype, device=qblk.device)
    _lib.call("rwkv_sb6_dequant", qblk.data_ptr(), qsqm.data_ptr(), ddm.data_ptr(), out.data_ptr(), _OUT_DT[dtype],
              out_features, in_features, xbits, _stream(qblk))
    return out


def rwkvq_dequant_sym(qblk, qs, d, out_features: int, in_features: int, bits: int,
                      dtype=torch.float32) -> torch.Tensor:
    """sym interleave → dense (RwkvqDequant.swift:409-431); shapes off the
    256-column super-block use the same kernel (the reference's op chain,
    :442-466, computes the same fp32 products)."""
    if dtype not in _OUT_DT:
        raise ValueError(f"sym dequant to {dtype} is not supported")
    qblk, qs, d = _sym_bufs(qblk, qs, d, out_features, in_features, bits)
    out = torch.empty((out_features, in_features), dtype=dtype, device=qblk.device)
    _lib.call("rwkv_sym_dequant", qblk.data_ptr(), qs.data_ptr(), d.data_ptr(), out.data_ptr(), _OUT_DT[dtype],
              out_features, in_features, bits, _stream(qblk))
    return out


def rwkvq_sym_rows(ids, qblk, qs, d, out_features: int, in_features: int, bits: int,
                   dtype=torch.float16) -> torch.Tensor:
    """Rows `ids` (any shape) of a sym matrix → [..., IN], dequantised on demand:
    bitwise the rows of rwkvq_dequant_sym (RwkvqSymRows.swift:43-53).  An id
    outside [0, OUT) gives a row of NaN."""
    if dtype not in _OUT_DT:
        raise ValueError(f"sym rows to {dtype} are not supported")
    qblk, qs, d = _sym_bufs(qblk, qs, d, out_features, in_features, bits)
    idx = ids.to(device=qblk.device, dtype=torch.int32).contiguous()
    out = torch.empty(tuple(idx.shape) + (in_features,), dtype=dtype, device=qblk.device)
    _lib.call("rwkv_sym_rows", idx.data_ptr(), idx.numel(), qblk.data_ptr(), qs.data_ptr(), d.data_ptr(),
              out.data_ptr(), _OUT_DT[dtype], out_features, in_features, bits, _stream(qblk))
    return out


def rwkvq_sb6_gemv_config(out_features: int, in_features: int, xbits: int) -> Tuple[int, int]:
    """(NSG, RS) table of the reference kernel (RwkvqSb6GEMV.swift:39-43).
    Only the applicability rule depends on it here."""
    if out_features >= 32768:
        return (4, 4)
    if out_features >= 8192:
        return (2, 2) if xbits == 0 else (4, 4)
    return (4, 4)


def rwkvq_sb6_gemv_applies(out_features: int, in_features: int, xbits: int, super_block: int, rows: int) -> bool:
    """RwkvqSb6GEMV.swift:159-164."""
    return bool(_lib.lib().rwkv_sb6_gemv_applies(out_features, in_features, xbits, super_block, rows))


def default_short_pass_rows(n_embd: int, sym: bool) -> int:
    """X070Backbone.defaultShortPassRows (X070Backbone.swift:384-389): up to
    this many input rows (B·T) a frozen parallel pass runs on the GEMV kernels.
    The reference's threshold reflects its one-row (sb6) / four-row (sym)
    launches; with every row in one launch the measured crossover is higher
    (bench.py reports it)."""
    return max(4, n_embd // (128 if sym else 256))


def rwkvq_sb6_gemv(x, qblk, qsqm, ddm, out_features: int, in_features: int, xbits: int,
                   out_per: Optional[int] = None) -> torch.Tensor:
    """y [N, OUT] = x [N, IN] · Wᵀ straight from the K3 bytes (RwkvqSb6GEMV.swift:170-190).
    The reference takes N = 1; here N rows share one weight pass.  With
    `out_per` (an extension: the reference fuses sym groups only) the K =
    OUT/out_per row-concatenated matrices run in one launch: x holds N·K rows
    and row o of input n reads x[n·K + o/out_per]."""
    if x.dim() != 2 or x.shape[1] != in_features:
        raise ValueError(f"sb6-GEMV: input {tuple(x.shape)}, expected [N, {in_features}]")
    per = out_features if out_per is None else out_per
    if per < 1 or out_features % per:
        raise ValueError(f"sb6-GEMV: {out_features} rows do not split into matrices of {per}")
    K = out_features // per
    if x.shape[0] % K:
        raise ValueError(f"sb6-GEMV: {x.shape[0]} input rows do not split over {K} fused matrices")
    N = x.shape[0] // K
    x32 = _aligned(x.to(torch.float32))
    qblk, qsqm, ddm = _sb6_bufs(qblk, qsqm, ddm, out_features, in_features, xbits)
    y = torch.empty((N, out_features), dtype=torch.float32, device=x.device)
    if out_per is None:
        _lib.call("rwkv_sb6_gemv", x32.data_ptr(), N, qblk.data_ptr(), qsqm.data_ptr(), ddm.data_ptr(),
                  y.data_ptr(), out_features, in_features, xbits, _stream(x32))
    else:
        _lib.call("rwkv_sb6_gemv_fused", x32.data_ptr(), N, qblk.data_ptr(), qsqm.data_ptr(), ddm.data_ptr(),
                  y.data_ptr(), out_features, in_features, xbits, per, _stream(x32))
    return y


RWKVQ_SYM_GEMV_MAX_ROWS = 4   # RwkvqSymGEMV.swift:40


def rwkvq_sym_gemv_applies(out_features: int, in_features: int, bits: int, rows: int) -> bool:
    """RwkvqSymGEMV.swift:213-218."""
    return bool(_lib.lib().rwkv_sym_gemv_applies(out_features, in_features, bits, rows))


def rwkvq_sym_gemv(x, qblk, qs, d, out_features: int, in_features: int, bits: int,
                   out_per: Optional[int] = None) -> torch.Tensor:
    """sym GEMV (RwkvqSymGEMV.swift:223-247); with `out_per` the K fused
    matrices of symGEMVFused (:343-358): x holds N·K rows, row o of input n
    reads x[n·K + o/out_per]."""
    if x.dim() != 2 or x.shape[1] != in_features:
        raise ValueError(f"sym-GEMV: input {tuple(x.shape)}, expected [N, {in_features}]")
    per = out_features if out_per is None else out_per
    K = out_features // per
    if x.shape[0] % K:
        raise ValueError(f"sym-GEMV: {x.shape[0]} input rows do not split over {K} fused matrices")
    N = x.shape[0] // K
    x32 = _aligned(x.to(torch.float32))
    qblk, qs, d = _sym_bufs(qblk, qs, d, out_features, in_features, bits)
    y = torch.empty((N, out_features), dtype=torch.float32, device=x.device)
    _lib.call("rwkv_sym_gemv", x32.data_ptr(), N, qblk.data_ptr(), qs.data_ptr(), d.data_ptr(), y.data_ptr(),
              out_features, in_features, bits, per, _stream(x32))
    return y


# ───────────────────────────── sidecar ─────────────────────────────

@dataclass
class RwkvqSb6FusedGroup:
    """Row-concatenated sb6 matrices of one fusion group (the sb6 counterpart
    of RwkvqSymFusedGroup)."""
    keys: List[str]
    qblk: torch.Tensor
    qsqm: torch.Tensor
    ddm: torch.Tensor
    out_per: int
    in_features: int
    xbits: int


@dataclass
class RwkvqSymRowTable:
    """An 8-bit sym embedding table read row by row; no dense table exists
    (RwkvqSymRows.swift:26-67)."""
    qblk: torch.Tensor
    qs: torch.Tensor
    d: torch.Tensor
    row_count: int
    in_features: int

    def rows(self, ids: torch.Tensor) -> torch.Tensor:
        """ids of any shape → [..., IN] fp16 (RwkvqSymRows.swift:43-53)."""
        return rwkvq_sym_rows(ids, self.qblk, self.qs, self.d, self.row_count, self.in_features, 8)

    def dense(self) -> torch.Tensor:
        """The whole table, [rows, IN] fp16 (RwkvqSymRows.swift:57-61)."""
        return rwkvq_dequant_sym(self.qblk, self.qs, self.d, self.row_count, self.in_features, 8, torch.float16)

    @property
    def packed_bytes(self) -> int:
        return self.qblk.numel() + self.qs.numel() + self.d.numel() * 2


@dataclass
class RwkvqSymFusedGroup:
    """RwkvqSymGEMV.swift:282-291."""
    keys: List[str]
    qblk: torch.Tensor
    qs: torch.Tensor
    d: torch.Tensor
    out_per: int
    in_features: int
    bits: int


class RwkvqSidecar:
    """Loaded quantised base: buffers + manifest (RwkvqSidecar.swift:102-132)."""

    max_format_version = 2

    def __init__(self, arrays: Dict[str, torch.Tensor], tensors: Dict[str, RwkvqTensorInfo], naming: str,
                 n_layer: int, n_embd: int, head_size: int, vocab_size: int,
                 sym_fused: Optional[Dict[str, RwkvqSymFusedGroup]] = None,
                 sb6_fused: Optional[Dict[str, RwkvqSb6FusedGroup]] = None):
        self.arrays = arrays
        self.tensors = tensors
        self.naming = naming
        self.n_layer, self.n_embd, self.head_size, self.vocab_size = n_layer, n_embd, head_size, vocab_size
        self.sym_fused = dict(sym_fused or {})
        self.sb6_fused = dict(sb6_fused or {})

    # RwkvqFile.swift:220-228
    @classmethod
    def open(cls, path: str, device="cuda") -> "RwkvqSidecar":
        return cls.from_rwkvq(path, device=device)

    @classmethod
    def from_rwkvq(cls, path: str, only: Optional[Callable[[str], bool]] = None,
                   fusing_sym: Optional[Dict[str, List[str]]] = None, device="cuda") -> "RwkvqSidecar":
        """Read a .rwkvq directly (RwkvqFile.swift:254-492): validate the whole
        manifest, load (and repack) the buffers of the tensors `only` admits."""
        p = os.path.expanduser(path)
        box = RwkvqContainer(p)
        text = box.metadata.get("rwkvq")
        try:
            root = json.loads(text) if text is not None else None
        except json.JSONDecodeError:
            root = None
        if not isinstance(root, dict):
            raise MalformedManifest(f"{p}: not .rwkvq — no rwkvq key in __metadata__")
        if root.get("format") != "rwkvq":
            raise MalformedManifest(f"{p}: format {root.get('format')}")
        version = root.get("format_version", 0)
        if not isinstance(version, int) or version > cls.max_format_version:
            raise MalformedManifest(f"{p}: format_version {version} newer than {cls.max_format_version}")
        tensor_dict = root.get("tensors")
        if not isinstance(tensor_dict, dict):
            raise MalformedManifest(f'{p}: no "tensors" section')
        naming = root.get("naming", "world")
        groups = dict(fusing_sym or {})
        arrays: Dict[str, torch.Tensor] = {}
        infos: Dict[str, RwkvqTensorInfo] = {}

        def to_dev(a: np.ndarray, as_t=None) -> torch.Tensor:
            t = torch.from_numpy(np.ascontiguousarray(a))
            if as_t is not None:
                t = t.view(as_t)
            return t.to(device)

        def process(key: str):
            m = tensor_dict.get(key)
            if not isinstance(m, dict) or not isinstance(m.get("shape"), list) or not isinstance(m.get("kind"), str):
                raise MalformedManifest(f"{p}: no shape or layout for {key}")
            try:
                kind = RwkvqKind(m["kind"])
            except ValueError:
                raise MalformedManifest(f"unknown layout {m['kind']} of {key}") from None
            shape = tuple(m["shape"])
            load = only(key) if only else True
            bits = m.get("bits", 16)
            gs = m.get("gw_gs", 0)
            sb = m.get("gw_sb", 0)
            transposed = m.get("transposed")
            if not isinstance(transposed, bool):
                transposed = naming == "world" and is_raw_lora_world(key)

            def need(field, as_dtype=None) -> np.ndarray:
                a = box.array(f"{key}::{field}", as_dtype)
                if a is None:
                    raise MissingBuffer(key, field)
                return a

            def dims(field) -> Tuple[int, ...]:
                s = box.shape(f"{key}::{field}")
                if s is None:
                    raise MissingBuffer(key, field)
                return s

            def n_blocks_check(got: int, what: str):
                nb = m.get("n_blocks")
                if isinstance(nb, int) and nb > 0 and nb != got:
                    raise MalformedManifest(f"{key}: {what} covers {got} blocks, the manifest says {nb}")

            xbits, packed, outliers = 0, False, 0
            if kind == RwkvqKind.dense:
                dims("dense")
                if load:
                    a = need("dense")
                    arrays[f"{key}::dense"] = (to_dev(a, torch.bfloat16) if box.dtype(f"{key}::dense") == "BF16"
                                               else to_dev(a))
            elif kind == RwkvqKind.asym:
                if len(shape) != 2 or gs <= 0:
                    raise MalformedManifest(f"incomplete asym entry for {key}")
                scale_shape = dims("gw_scale")
                nb = (shape[1] + gs - 1) // gs
                if not scale_shape or scale_shape[-1] != nb:
                    raise ShapeMismatch(key, [shape[0], nb], scale_shape)
                n_blocks_check(nb, "gw_scale")
                dims("codes")
                dims("gw_min")
                if load:
                    for f in ("codes", "gw_scale", "gw_min"):
                        arrays[f"{key}::{f}"] = to_dev(need(f))
            elif kind == RwkvqKind.rtn:
                packed = box.contains(f"{key}::codes_packed")
                if not packed:
                    dims("codes")
                dims("scale")
                if load:
                    f = "codes_packed" if packed else "codes"
                    arrays[f"{key}::{f}"] = to_dev(need(f))
                    arrays[f"{key}::scale"] = to_dev(need("scale"))
                os_ = box.shape(f"{key}::outlier_indices")
                outliers = os_[0] if os_ else 0
            elif kind == RwkvqKind.sb6:
                if not (len(shape) == 2 and gs == 32 and sb == 8 and shape[1] % (gs * sb) == 0):
                    raise MalformedManifest(
                        f"{key}: sb6 is read with block 32 and super-block 8 (file: gw_gs={gs}, gw_sb={sb}, shape {list(shape)})")
                n_blocks_check(shape[1] // gs, "sb6")
                want = (shape[0], shape[1] // (gs * sb), 12)
                got = dims("gw_qsqm")
                if tuple(got) != want:
                    raise ShapeMismatch(key, want, got)
                dims("codes_packed")
                dims("gw_d")
                dims("gw_dm")
                xbits = int(box.contains(f"{key}::gw_qh")) + int(box.contains(f"{key}::gw_qh2"))
                if bits != 4 + xbits:
                    raise MalformedManifest(f"{key}: bits={bits}, but the file has {xbits} bit planes")
                if load:
                    qblk, k3, ddm, xb = rwkvq_sb6_to_k3(
                        need("codes_packed"), need("gw_qsqm"), need("gw_d", np.uint16), need("gw_dm", np.uint16),
                        box.array(f"{key}::gw_qh"), box.array(f"{key}::gw_qh2"), shape, gs, sb)
                    assert xb == xbits
                    arrays[f"{key}::qblk"] = to_dev(qblk)
                    arrays[f"{key}::qsqm"] = to_dev(k3)
                    arrays[f"{key}::ddm"] = to_dev(ddm, torch.float16)
            elif kind == RwkvqKind.sym:
                if not (len(shape) == 2 and gs == 16 and sb == 16):
                    raise MalformedManifest(f"{key}: sym is read with block 16 and super-block 16 (file: gw_gs={gs}, gw_sb={sb})")
                OUT, IN = shape
                if IN % gs:
                    raise MalformedManifest(f"{key}: sym, IN={IN} is not a multiple of block 16")
                qs_shape, d_shape = dims("gw_qs"), dims("gw_d")
                n_blocks_check(qs_shape[-1] if qs_shape else 0, "gw_qs")
                if tuple(qs_shape) != (OUT, IN // gs) or len(d_shape) != 2 or d_shape[1] * sb != IN // gs:
                    raise ShapeMismatch(key, [OUT, IN // gs], qs_shape)
                eight = box.contains(f"{key}::codes")
                if eight:
                    if bits != 8:
                        raise MalformedManifest(f"{key}: sym with a codes buffer at bits={bits}")
                else:
                    if bits != 6 or IN % 32:
                        raise MalformedManifest(f"{key}: sym with codes_packed at bits={bits}, IN={IN}")
                    dims("codes_packed")
                    dims("gw_qh")
                    dims("gw_qh2")
                if load:
                    if eight:
                        qblk = need("codes", np.uint8)
                    else:
                        qblk = rwkvq_sym_interleave(need("codes_packed"), need("gw_qh"), need("gw_qh2"), shape)
                    arrays[f"{key}::qblk"] = to_dev(qblk)
                    arrays[f"{key}::qs"] = to_dev(need("gw_qs", np.uint8))
                    arrays[f"{key}::d"] = to_dev(need("gw_d", np.uint16), torch.float16)
            infos[key] = RwkvqTensorInfo(kind=kind, shape=shape, bits=bits, xbits=xbits, group_size=gs,
                                         super_block=sb, packed=packed, outlier_count=outliers,
                                         transposed=transposed)

        def elements(key):
            m = tensor_dict.get(key)
            s = m.get("shape", []) if isinstance(m, dict) else []
            n = 1
            for v in s:
                n *= v
            return n

        group_of = {k: gid for gid, keys in groups.items() for k in keys}
        fused: Dict[str, RwkvqSymFusedGroup] = {}
        done = set()
        ordered = sorted(tensor_dict.keys(), key=lambda k: (-elements(k), k))
        for key in ordered:
            if key in done:
                continue
            gid = group_of.get(key)
            members = groups.get(gid) if gid is not None else None
            if members is None or not all(k in tensor_dict and (only(k) if only else True) for k in members):
                process(key)
                done.add(key)
                continue
            for k in members:
                if k not in done:
                    process(k)
                    done.add(k)
            g = _fuse_sym_group(members, infos, arrays)
            if g is not None:
                fused[gid] = g
        box.close()
        return cls(arrays, infos, naming, root.get("n_layer", 0), root.get("n_embd", 0),
                   root.get("head_size", 64), root.get("vocab_size", 0), fused)

    # ── queries ──
    @property
    def keys(self) -> List[str]:
        return sorted(self.tensors)

    def contains(self, key: str) -> bool:
        return key in self.tensors

    def pruned(self, keeping: Iterable[str]) -> "RwkvqSidecar":
        """RwkvqSidecar.swift:215-225."""
        keep = set(keeping)
        a = {n: v for n, v in self.arrays.items() if n.split("::", 1)[0] in keep}
        return RwkvqSidecar(a, {k: v for k, v in self.tensors.items() if k in keep}, self.naming, self.n_layer,
                            self.n_embd, self.head_size, self.vocab_size,
                            {g: v for g, v in self.sym_fused.items() if all(k in keep for k in v.keys)},
                            {g: v for g, v in self.sb6_fused.items() if all(k in keep for k in v.keys)})

    @property
    def packed_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.arrays.values())

    def _buf(self, key: str, field: str) -> torch.Tensor:
        t = self.arrays.get(f"{key}::{field}")
        if t is None:
            raise MissingBuffer(key, field)
        return t

    def dequantize(self, key: str, dtype=torch.float32) -> torch.Tensor:
        """Any layout → dense, in the stored orientation (RwkvqSidecar.swift:243-325)."""
        info = self.tensors.get(key)
        if info is None:
            raise MissingBuffer(key, "manifest")
        if info.kind == RwkvqKind.dense:
            return self._buf(key, "dense").to(dtype)
        if info.kind == RwkvqKind.sb6:
            return rwkvq_dequant_dense(self._buf(key, "qblk"), self._buf(key, "qsqm"), self._buf(key, "ddm"),
                                       info.out_features, info.in_features, info.super_block, info.xbits, dtype)
        if info.kind == RwkvqKind.sym:
            return rwkvq_dequant_sym(self._buf(key, "qblk"), self._buf(key, "qs"), self._buf(key, "d"),
                                     info.out_features, info.in_features, info.bits, dtype)
        if info.kind == RwkvqKind.asym:
            codes, scale, mn = self._buf(key, "codes"), self._buf(key, "gw_scale"), self._buf(key, "gw_min")
            return rwkvq_dequant_asym(codes, scale, mn, info.group_size, dtype)
        # rtn
        if info.packed:
            codes = rwkvq_unpack_int4(self._buf(key, "codes_packed"), info.in_features)
        else:
            codes = self._buf(key, "codes")
        scale = self._buf(key, "scale")
        if info.outlier_count > 0:
            raise UnsupportedKind(key, "rtn+outliers (SpQR scatter not implemented)")
        return rwkvq_dequant_rtn(codes, scale, dtype)

    def build_dense_weights(self, dtype=torch.float16) -> Dict[str, torch.Tensor]:
        """The x070 dictionary of everything but the quantised projections
        (RwkvqSidecar.buildDenseWeights, RwkvqFullConvert.swift:49-140): layer
        norms, token-shift coefficients, k_k / k_a / r_k as [H, S], the
        low-rank branches in the Linear convention (A [rank, D], B [D, rank];
        a tensor whose manifest says `transposed` is turned, and the shape is
        checked), w0 / a0 / v0 flattened into the B biases, the v branch only
        for layers > 0, ln_x and the cmix coefficient; plus `emb.weight`
        dequantised once (load(fromSidecar:), X070Backbone.swift)."""
        if not (self.n_layer > 0 and self.n_embd > 0 and self.head_size > 0):
            raise IncompleteManifest("n_layer / n_embd / head_size missing or zero: the manifest does not describe "
                                     "the model")
        if not any(t.kind == RwkvqKind.dense for t in self.tensors.values()):
            raise PartialExport(len(self.tensors))
        D, S = self.n_embd, self.head_size
        H = D // S
        dq = lambda k: self.dequantize(k, dtype)

        def low_rank(k: str, is_a: bool) -> torch.Tensor:
            info = self.tensors.get(k)
            if info is None:
                raise MissingBuffer(k, "manifest")
            v = dq(k)
            if info.transposed:
                v = v.t().contiguous()
            if v.dim() != 2 or v.shape[1 if is_a else 0] != D:
                raise ShapeMismatch(k, [-1, D] if is_a else [D, -1], list(v.shape))
            return v

        out = {"ln0.weight": dq("blocks.0.ln0.weight"), "ln0.bias": dq("blocks.0.ln0.bias"),
               "ln_out.weight": dq("ln_out.weight"), "ln_out.bias": dq("ln_out.bias")}
        for i in range(self.n_layer):
            b = f"blocks.{i}."
            att, ffn, P = b + "att.", b + "ffn.", b + "tmix."
            for n in ("ln1", "ln2"):
                out[b + n + ".weight"] = dq(b + n + ".weight")
                out[b + n + ".bias"] = dq(b + n + ".bias")
            for x in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"):
                out[P + x] = dq(att + x)
            for x in ("k_k", "k_a", "r_k"):
                out[P + x] = dq(att + x).reshape(H, S)
            branches = [("w", True), ("a", True), ("g", False)] + ([("v", True)] if i > 0 else [])
            for n, bias in branches:
                out[P + n + "_lora_A.weight"] = low_rank(att + n + "1", True)
                out[P + n + "_lora_B.weight"] = low_rank(att + n + "2", False)
                if bias:
                    out[P + n + "_lora_B.bias"] = dq(att + n + "0").reshape(D)
            out[P + "ln_x.weight"] = dq(att + "ln_x.weight")
            out[P + "ln_x.bias"] = dq(att + "ln_x.bias")
            out[b + "cmix.x_k"] = dq(ffn + "x_k")
        out["emb.weight"] = dq("emb.weight")
        return out

    def sym_row_table(self, key: str) -> Optional[RwkvqSymRowTable]:
        """RwkvqSymRows.swift:70-80: a row table for an 8-bit sym tensor, None
        otherwise (the caller then takes the dense path)."""
        info = self.tensors.get(key)
        if (info is None or info.kind != RwkvqKind.sym or info.bits != 8 or len(info.shape) != 2
                or info.in_features % 16):
            return None
        names = [f"{key}::{f}" for f in ("qblk", "qs", "d")]
        if any(n not in self.arrays for n in names):
            return None
        qblk, qs, d = (self.arrays[n] for n in names)
        return RwkvqSymRowTable(qblk, qs, d, info.out_features, info.in_features)

    # ── projections (the .rwkvq branch of the model's baseProj) ──
    def base_proj(self, key: str, x: torch.Tensor, base_dtype=torch.float16, decode: bool = False,
                  short_rows: int = 0) -> torch.Tensor:
        """x [..., IN] · Wᵀ → [..., OUT] in x's dtype, the .rwkvq branch of
        X070Backbone.baseProj (X070Backbone.swift:676-746, 337-341): on the
        recurrent step (`decode`) or a short parallel pass (B·T ≤ `short_rows`,
        RWKVBlock.swift:418-423) the GEMV kernel on the packed codes; otherwise
        dequantise to `base_dtype` and matmul in it.  The reference splits the
        GEMV rows into launches of one (sb6) or four (sym); here all rows go in
        one launch."""
        info = self.tensors.get(key)
        if info is None:
            raise MissingBuffer(key, "manifest")
        IN, OUT = info.in_features, info.out_features
        if x.shape[-1] != IN:
            raise ValueError(f"base_proj {key}: input {tuple(x.shape)}, expected [..., {IN}]")
        lead = tuple(x.shape[:-1])
        x2d = x.reshape(-1, IN)
        rows = x2d.shape[0]
        if decode or (short_rows > 0 and rows <= short_rows):
            y = None
            if info.kind == RwkvqKind.sb6 and rwkvq_sb6_gemv_applies(OUT, IN, info.xbits, info.super_block, 1):
                y = rwkvq_sb6_gemv(x2d.float(), self._buf(key, "qblk"), self._buf(key, "qsqm"),
                                   self._buf(key, "ddm"), OUT, IN, info.xbits)
            elif info.kind == RwkvqKind.sym and rwkvq_sym_gemv_applies(OUT, IN, info.bits, 1):
                y = rwkvq_sym_gemv(x2d.float(), self._buf(key, "qblk"), self._buf(key, "qs"), self._buf(key, "d"),
                                   OUT, IN, info.bits)
            if y is not None:
                return y.to(x.dtype).reshape(*lead, OUT)
        W = self.dequantize(key, base_dtype)   # the transient dense weight, [OUT, IN]
        y = torch.nn.functional.linear(x2d.to(base_dtype), W)
        return y.to(x.dtype).reshape(*lead, OUT)

    # ── GEMV (decode) ──
    def sb6_gemv(self, key: str, x: torch.Tensor) -> Optional[torch.Tensor]:
        """RwkvqSb6GEMV.swift:197-208: None when the kernel does not take it."""
        info = self.tensors.get(key)
        if (info is None or info.kind != RwkvqKind.sb6 or x.dim() != 2 or x.shape[1] != info.in_features
                or not rwkvq_sb6_gemv_applies(info.out_features, info.in_features, info.xbits, info.super_block,
                                              x.shape[0])):
            return None
        names = [f"{key}::{f}" for f in ("qblk", "qsqm", "ddm")]
        if any(n not in self.arrays for n in names):
            return None
        return rwkvq_sb6_gemv(x, *[self.arrays[n] for n in names], info.out_features, info.in_features, info.xbits)

    def sym_gemv(self, key: str, x: torch.Tensor) -> Optional[torch.Tensor]:
        """RwkvqSymGEMV.swift:254-263."""
        info = self.tensors.get(key)
        if (info is None or info.kind != RwkvqKind.sym or x.dim() != 2 or x.shape[1] != info.in_features
                or not rwkvq_sym_gemv_applies(info.out_features, info.in_features, info.bits, x.shape[0])):
            return None
        names = [f"{key}::{f}" for f in ("qblk", "qs", "d")]
        if any(n not in self.arrays for n in names):
            return None
        return rwkvq_sym_gemv(x, *[self.arrays[n] for n in names], info.out_features, info.in_features, info.bits)

    def fusing_sym(self, groups: Dict[str, List[str]]) -> "RwkvqSidecar":
        """Concatenate the rows of each sym group into one buffer; the member
        buffers become row slices of it (RwkvqSymGEMV.swift:298-310)."""
        a = dict(self.arrays)
        fused = dict(self.sym_fused)
        for gid, keys in groups.items():
            if gid in fused:
                continue
            g = _fuse_sym_group(keys, self.tensors, a)
            if g is not None:
                fused[gid] = g
        return RwkvqSidecar(a, dict(self.tensors), self.naming, self.n_layer, self.n_embd, self.head_size,
                            self.vocab_size, fused, self.sb6_fused)

    def fusing_sb6(self, groups: Dict[str, List[str]]) -> "RwkvqSidecar":
        """fusing_sym for sb6 groups (an extension: r/k/v of an sb6 model in
        one launch).  Member buffers become row slices of the group buffer."""
        a = dict(self.arrays)
        fused = dict(self.sb6_fused)
        for gid, keys in groups.items():
            if gid in fused:
                continue
            g = _fuse_sb6_group(keys, self.tensors, a)
            if g is not None:
                fused[gid] = g
        return RwkvqSidecar(a, dict(self.tensors), self.naming, self.n_layer, self.n_embd, self.head_size,
                            self.vocab_size, self.sym_fused, fused)

    def sb6_gemv_fused(self, gid: str, xstack: torch.Tensor) -> Optional[torch.Tensor]:
        """K sb6 projections in one launch: xstack [K, IN] → [K, out_per]."""
        g = self.sb6_fused.get(gid)
        if g is None or xstack.dim() != 2 or tuple(xstack.shape) != (len(g.keys), g.in_features):
            return None
        K = len(g.keys)
        y = rwkvq_sb6_gemv(xstack, g.qblk, g.qsqm, g.ddm, g.out_per * K, g.in_features, g.xbits, out_per=g.out_per)
        return y.reshape(K, g.out_per)

    def sym_gemv_fused(self, gid: str, xstack: torch.Tensor) -> Optional[torch.Tensor]:
        """K projections in one launch: xstack [K, IN] → [K, out_per] (RwkvqSymGEMV.swift:343-358)."""
        g = self.sym_fused.get(gid)
        if g is None or xstack.dim() != 2 or tuple(xstack.shape) != (len(g.keys), g.in_features):
            return None
        K = len(g.keys)
        y = rwkvq_sym_gemv(xstack, g.qblk, g.qs, g.d, g.out_per * K, g.in_features, g.bits, out_per=g.out_per)
        return y.reshape(K, g.out_per)


def _fuse_sb6_group(keys: List[str], tensors: Dict[str, RwkvqTensorInfo],
                    arrays: Dict[str, torch.Tensor]) -> Optional[RwkvqSb6FusedGroup]:
    """sb6 counterpart of _fuse_sym_group: same shape and xbits, every member
    taken by the sb6 GEMV.  None (arrays untouched) when the group does not
    qualify."""
    if len(keys) < 2:
        return None
    first = tensors.get(keys[0])
    if first is None or first.kind != RwkvqKind.sb6:
        return None
    for k in keys:
        t = tensors.get(k)
        if (t is None or t.kind != RwkvqKind.sb6 or t.shape != first.shape or t.xbits != first.xbits
                or t.super_block != first.super_block
                or any(f"{k}::{f}" not in arrays for f in ("qblk", "qsqm", "ddm"))):
            return None
    if not rwkvq_sb6_gemv_applies(first.out_features, first.in_features, first.xbits, first.super_block, 1):
        return None
    OUT = first.out_features
    cat = {f: torch.cat([arrays[f"{k}::{f}"] for k in keys], 0) for f in ("qblk", "qsqm", "ddm")}
    for i, k in enumerate(keys):
        for f in ("qblk", "qsqm", "ddm"):
            arrays[f"{k}::{f}"] = cat[f][i * OUT:(i + 1) * OUT]
    return RwkvqSb6FusedGroup(list(keys), cat["qblk"], cat["qsqm"], cat["ddm"], OUT, first.in_features, first.xbits)


def _fuse_sym_group(keys: List[str], tensors: Dict[str, RwkvqTensorInfo],
                    arrays: Dict[str, torch.Tensor]) -> Optional[RwkvqSymFusedGroup]:
    """RwkvqSymGEMV.swift:314-339.  Returns None (arrays untouched) when the
    group does not qualify."""
    if len(keys) < 2:
        return None
    first = tensors.get(keys[0])
    if first is None or first.kind != RwkvqKind.sym:
        return None
    for k in keys:
        t = tensors.get(k)
        if (t is None or t.kind != RwkvqKind.sym or t.shape != first.shape or t.bits != first.bits
                or any(f"{k}::{f}" not in arrays for f in ("qblk", "qs", "d"))):
            return None
    if not rwkvq_sym_gemv_applies(first.out_features * len(keys), first.in_features, first.bits, 1) \
            or first.out_features % 4:
        return None
    OUT = first.out_features
    qblk = torch.cat([arrays[f"{k}::qblk"] for k in keys], 0)
    qs = torch.cat([arrays[f"{k}::qs"] for k in keys], 0)
    d = torch.cat([arrays[f"{k}::d"] for k in keys], 0)
    for i, k in enumerate(keys):
        arrays[f"{k}::qblk"] = qblk[i * OUT:(i + 1) * OUT]
        arrays[f"{k}::qs"] = qs[i * OUT:(i + 1) * OUT]
        arrays[f"{k}::d"] = d[i * OUT:(i + 1) * OUT]
    return RwkvqSymFusedGroup(list(keys), qblk, qs, d, OUT, first.in_features, first.bits)


# ───────────────────────────── asym / rtn (op chains, as in the reference) ─────────────────────────────

def rwkvq_dequant_asym(codes, scale, mn, group_size: int, dtype=torch.float32) -> torch.Tensor:
    """RwkvqDequant.swift:197-212 (an op chain there too, not a kernel)."""
    IN = codes.shape[1]
    idx = torch.arange(IN, device=codes.device) // group_size
    s = scale.to(torch.float32).index_select(1, idx)
    m = mn.to(torch.float32).index_select(1, idx)
    return (codes.to(torch.float32) * s + m).to(dtype)


def rwkvq_dequant_rtn(codes, scale, dtype=torch.float32) -> torch.Tensor:
    """RwkvqDequant.swift:218-222."""
    return (codes.to(torch.float32) * scale.to(torch.float32)).to(dtype)


def rwkvq_unpack_int4(packed, columns: int) -> torch.Tensor:
    """RwkvqDequant.swift:228-233: biased split nibble layout."""
    p = packed.to(torch.int32)
    lo = (p & 0x0F) - 8
    hi = (p >> 4) - 8
    return torch.cat([lo, hi], 1)[:, :columns].to(torch.int8)


# ───────────────────────────── encoders / writer (not in the reference) ─────────────────────────────

def encode_sb6(w: np.ndarray, bits: int = 4, nthreads: int = 8) -> Dict[str, np.ndarray]:
    """Quantise fp32 [OUT, IN] to the sb6 DISK layout (codes_packed, gw_qh,
    gw_qh2, gw_qsqm, gw_d, gw_dm).  Encoder calibration is this project's own."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    OUT, IN = w.shape
    NB, NSB = IN // 32, IN // 256
    out = {"codes_packed": np.empty((OUT, NB * 16), np.uint8),
           "gw_qsqm": np.empty((OUT, NSB, 12), np.uint8),
           "gw_d": np.empty((OUT, NSB), np.float16),
           "gw_dm": np.empty((OUT, NSB), np.float16)}
    if bits >= 5:
        out["gw_qh"] = np.empty((OUT, NB * 4), np.uint8)
    if bits >= 6:
        out["gw_qh2"] = np.empty((OUT, NB * 4), np.uint8)
    _lib.call("rwkvq_encode_sb6", _np_ptr(w), OUT, IN, bits, _np_ptr(out["codes_packed"]), _np_ptr(out.get("gw_qh")),
              _np_ptr(out.get("gw_qh2")), _np_ptr(out["gw_qsqm"]), _np_ptr(out["gw_d"]), _np_ptr(out["gw_dm"]),
              nthreads)
    return out


def encode_sym(w: np.ndarray, bits: int = 8, nthreads: int = 8) -> Dict[str, np.ndarray]:
    """Quantise fp32 [OUT, IN] to the sym DISK layout (codes | codes_packed +
    gw_qh + gw_qh2, gw_qs, gw_d)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    OUT, IN = w.shape
    out = {"gw_qs": np.empty((OUT, IN // 16), np.int8), "gw_d": np.empty((OUT, IN // 256), np.float16)}
    if bits == 8:
        out["codes"] = np.empty((OUT, IN), np.int8)
    else:
        out["codes_packed"] = np.empty((OUT, IN // 32 * 16), np.uint8)
        out["gw_qh"] = np.empty((OUT, IN // 32 * 4), np.uint8)
        out["gw_qh2"] = np.empty((OUT, IN // 32 * 4), np.uint8)
    _lib.call("rwkvq_encode_sym", _np_ptr(w), OUT, IN, bits, _np_ptr(out.get("codes")),
              _np_ptr(out.get("codes_packed")), _np_ptr(out.get("gw_qh")), _np_ptr(out.get("gw_qh2")),
              _np_ptr(out["gw_qs"]), _np_ptr(out["gw_d"]), nthreads)
    return out


_NP_ST = {np.dtype(np.uint8): "U8", np.dtype(np.int8): "I8", np.dtype(np.float16): "F16",
          np.dtype(np.float32): "F32", np.dtype(np.int32): "I32", np.dtype(np.uint16): "U16",
          np.dtype(np.int64): "I64", np.dtype(np.float64): "F64", np.dtype(np.bool_): "BOOL"}


def write_safetensors(path: str, buffers: Dict[str, np.ndarray], metadata: Optional[Dict[str, str]] = None,
                      dtypes: Optional[Dict[str, str]] = None) -> None:
    """Plain safetensors writer (u64-LE header length, JSON header padded to
    8 bytes, raw little-endian data).  `dtypes` overrides a buffer's
    safetensors dtype name (e.g. "BF16" for uint16 bit patterns)."""
    header = {}
    if metadata:
        header["__metadata__"] = dict(metadata)
    off = 0
    names = sorted(buffers)
    for n in names:
        a = np.ascontiguousarray(buffers[n])
        dt = (dtypes or {}).get(n) or _NP_ST[a.dtype]
        header[n] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        off += a.nbytes
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * ((8 - len(hb) % 8) % 8)
    with open(path, "wb") as f:
        f.write(len(hb).to_bytes(8, "little"))
        f.write(hb)
        for n in names:
            f.write(np.ascontiguousarray(buffers[n]).tobytes())


def write_rwkvq(path: str, tensors: Dict[str, Tuple[dict, Dict[str, np.ndarray]]], *, n_layer: int = 0,
                n_embd: int = 0, head_size: int = 64, vocab_size: int = 0, naming: str = "world",
                format_version: int = 2) -> None:
    """Write a .rwkvq: `tensors` maps key → (manifest entry, {field: buffer})."""
    manifest = {"format": "rwkvq", "format_version": format_version, "naming": naming, "n_layer": n_layer,
                "n_embd": n_embd, "head_size": head_size, "vocab_size": vocab_size,
                "tensors": {k: m for k, (m, _) in tensors.items()}}
    bufs = {f"{k}::{f}": a for k, (_, fields) in tensors.items() for f, a in fields.items()}
    write_safetensors(path, bufs, {"rwkvq": json.dumps(manifest)})


def sb6_entry(w: np.ndarray, bits: int = 4, nthreads: int = 8):
    """(manifest entry, disk buffers) of one sb6 tensor."""
    OUT, IN = w.shape
    return ({"kind": "sb6", "shape": [OUT, IN], "bits": bits, "xbits": bits - 4, "gw_gs": 32, "gw_sb": 8,
             "n_blocks": IN // 32}, encode_sb6(w, bits, nthreads))


def sym_entry(w: np.ndarray, bits: int = 8, nthreads: int = 8):
    OUT, IN = w.shape
    return ({"kind": "sym", "shape": [OUT, IN], "bits": bits, "gw_gs": 16, "gw_sb": 16}, encode_sym(w, bits, nthreads))
