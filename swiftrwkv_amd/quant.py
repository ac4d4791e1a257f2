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
    def __init__(self, tensor: str, buffer: str, message: Optional[str] = None):
        self.tensor, self.buffer = tensor, buffer
        super().__init__(message or f"no buffer {buffer} for tensor {tensor}")


class ShapeMismatch(RwkvqError):
    def __init__(self, tensor: str, expected, got, message: Optional[str] = None):
        self.tensor, self.expected, self.got = tensor, list(expected), list(got)
        super().__init__(message or f"{tensor}: expected shape {self.expected}, file has {self.got}")


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


# ───────────────────────────── manifest ─────────────────────────────

_KINDS = (RwkvqKind.dense, RwkvqKind.sb6, RwkvqKind.sym, RwkvqKind.asym, RwkvqKind.rtn)   # rwkvq_kind order


class RwkvqManifest:
    """The .rwkvq manifest of an open container, checked by the C reader
    (rwkvq_manifest_read) as a whole before anything is loaded: the tensor
    table (key → RwkvqTensorInfo) and the model fields.  Lives as long as
    the container it was read from."""

    def __init__(self, box: RwkvqContainer, max_format_version: int):
        lib = _lib.lib()
        h, finding = ctypes.c_void_p(), _lib.Finding()
        st = lib.rwkvq_manifest_read(box._h, max_format_version, ctypes.byref(h), ctypes.byref(finding))
        if st != _lib.RWKV_OK:
            raise _finding_error(finding, lib.rwkv_last_error().decode())
        self._box, self._h = box, h
        model = _lib.ModelDesc()
        _lib.check(lib.rwkvq_manifest_model(h, ctypes.byref(model)))
        self.format_version = model.format_version
        self.naming = model.naming.decode()
        self.n_layer, self.n_embd = model.n_layer, model.n_embd
        self.head_size, self.vocab_size = model.head_size, model.vocab_size
        self.infos: Dict[str, RwkvqTensorInfo] = {}
        self._index: Dict[str, int] = {}
        d = _lib.TensorDesc()
        for i in range(lib.rwkvq_manifest_count(h)):
            _lib.check(lib.rwkvq_manifest_tensor(h, i, ctypes.byref(d)))
            key = d.key.decode()
            self._index[key] = i
            self.infos[key] = RwkvqTensorInfo(
                kind=_KINDS[d.kind], shape=tuple(d.shape[j] for j in range(d.ndim)), bits=d.bits, xbits=d.xbits,
                group_size=d.group_size, super_block=d.super_block, packed=bool(d.packed),
                outlier_count=d.outliers, transposed=bool(d.transposed))

    def __del__(self):
        if getattr(self, "_h", None):
            _lib.lib().rwkvq_manifest_free(self._h)
            self._h = None

    @property
    def keys(self) -> List[str]:
        return list(self.infos)

    def buffer(self, key: str, field: str, as_dtype=None) -> np.ndarray:
        """A buffer of an entry, as stored (the dense / asym / rtn op-chain inputs)."""
        return self._box.array(f"{key}::{field}", as_dtype)

    def read_into(self, key: str, bufs: Tuple[np.ndarray, ...]) -> None:
        """The loader layout of an sb6 / sym matrix into (qblk, qsqm|qs, ddm|d):
        contiguous host arrays, or row slices of a group's arrays."""
        info = self.infos[key]
        fn = "rwkvq_read_sb6" if info.kind == RwkvqKind.sb6 else "rwkvq_read_sym"
        _lib.call(fn, self._box._h, self._h, self._index[key], *[_np_ptr(b) for b in bufs])


def _finding_error(f: "_lib.Finding", message: str) -> RwkvqError:
    tensor, buffer = f.tensor.decode(), f.buffer.decode()
    if f.kind == 2:
        return MissingBuffer(tensor, buffer, message)
    if f.kind == 3:
        return ShapeMismatch(tensor, f.expected[:f.n_expected], f.got[:f.n_got], message)
    return MalformedManifest(message)


def _loader_arrays(info: RwkvqTensorInfo, rows: int) -> Tuple[np.ndarray, ...]:
    """Host arrays for `rows` rows of an sb6 / sym matrix in the loader layouts."""
    IN = info.in_features
    if info.kind == RwkvqKind.sb6:
        return (np.empty((rows, IN // 32 * (16 + 4 * info.xbits)), np.uint8), np.empty((rows, IN // 16), np.uint8),
                np.empty((rows, IN // 128), np.uint16))
    width = IN if info.bits == 8 else IN // 32 * 24
    return np.empty((rows, width), np.uint8), np.empty((rows, IN // 16), np.uint8), np.empty((rows, IN // 256), np.uint16)


def _loader_fields(kind: RwkvqKind) -> Tuple[str, str, str]:
    return ("qblk", "qsqm", "ddm") if kind == RwkvqKind.sb6 else ("qblk", "qs", "d")


def _to_device(a: np.ndarray, device, as_torch=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a))
    if as_torch is not None:
        t = t.view(as_torch)
    return t.to(device)


def _read_tensor(man: RwkvqManifest, key: str, device) -> Dict[str, torch.Tensor]:
    """The device buffers one entry is kept in (names "<key>::<field>")."""
    info = man.infos[key]
    if info.is_quantized_base:
        host = _loader_arrays(info, info.out_features)
        man.read_into(key, host)
        fields = _loader_fields(info.kind)
        return {f"{key}::{f}": _to_device(a, device, torch.float16 if a.dtype == np.uint16 else None)
                for f, a in zip(fields, host)}
    if info.kind == RwkvqKind.dense:
        raw = man.buffer(key, "dense")
        bf16 = man._box.dtype(f"{key}::dense") == "BF16"
        return {f"{key}::dense": _to_device(raw, device, torch.bfloat16 if bf16 else None)}
    fields = ("codes", "gw_scale", "gw_min") if info.kind == RwkvqKind.asym else (
        ("codes_packed" if info.packed else "codes"), "scale")
    return {f"{key}::{f}": _to_device(man.buffer(key, f), device) for f in fields}


def _sym_fusable(members: List[RwkvqTensorInfo]) -> bool:
    """The sym fusion condition (RwkvqSymGEMV.swift:314-339): ≥ 2 sym matrices
    of one shape and code width whose row-concatenation the sym GEMV takes,
    with a whole number of its 4-row groups per matrix."""
    if len(members) < 2 or any(m is None or m.kind != RwkvqKind.sym for m in members):
        return False
    m0 = members[0]
    if any(m.shape != m0.shape or m.bits != m0.bits for m in members):
        return False
    return rwkvq_sym_gemv_applies(m0.out_features * len(members), m0.in_features, m0.bits, 1) and \
        m0.out_features % 4 == 0


def _plan_fused_reads(groups: Dict[str, List[str]], infos: Dict[str, RwkvqTensorInfo],
                      admitted: set) -> Dict[str, List[str]]:
    """The groups to read as one buffer: every member admitted and the
    group fusable; a key joins at most one group (the first that claims it)."""
    plan, claimed = {}, set()
    for gid, keys in groups.items():
        if any(k not in admitted or k in claimed for k in keys):
            continue
        if _sym_fusable([infos.get(k) for k in keys]):
            plan[gid] = list(keys)
            claimed.update(keys)
    return plan


def _read_sym_group(man: RwkvqManifest, keys: List[str], arrays: Dict[str, torch.Tensor],
                    device) -> "RwkvqSymFusedGroup":
    """Reads the members into row ranges of one set of host arrays, moves it
    to the device once, and files each member as a row view."""
    info = man.infos[keys[0]]
    OUT = info.out_features
    host = _loader_arrays(info, OUT * len(keys))
    for i, k in enumerate(keys):
        man.read_into(k, tuple(a[i * OUT:(i + 1) * OUT] for a in host))
    dev = [_to_device(a, device, torch.float16 if a.dtype == np.uint16 else None) for a in host]
    for i, k in enumerate(keys):
        for f, t in zip(_loader_fields(info.kind), dev):
            arrays[f"{k}::{f}"] = t[i * OUT:(i + 1) * OUT]
    return RwkvqSymFusedGroup(list(keys), dev[0], dev[1], dev[2], OUT, info.in_features, info.bits)


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
    need = (OUT * IN // 2, OUT * IN // 8, OUT * IN // 8, OUT * (IN // 256) * 12, OUT * (IN // 256), OUT * (IN // 256))
    for name, x, n in zip(("codes_packed", "qh", "qh2", "qsqm", "d", "dm"), c, need):
        if x is not None and x.size != n:
            raise ValueError(f"sb6 repack: {name} holds {x.size} elements, [{OUT}, {IN}] needs {n}")
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
    for name, x, n in zip(("codes_packed", "qh", "qh2"), c, (OUT * IN // 2, OUT * IN // 8, OUT * IN // 8)):
        if x.size != n:
            raise ValueError(f"sym interleave: {name} holds {x.size} bytes, [{OUT}, {IN}] needs {n}")
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


def rwkvq_sb6_gemm_applies(out_features: int, in_features: int, xbits: int, out_per: Optional[int] = None) -> bool:
    """Whether the matrix-core long pass takes this sb6 matrix (group)."""
    per = out_features if out_per is None else out_per
    return bool(_lib.lib().rwkv_sb6_gemm_applies(out_features, in_features, xbits, per))


def rwkvq_sym_gemm_applies(out_features: int, in_features: int, bits: int, out_per: Optional[int] = None) -> bool:
    """Whether the matrix-core long pass takes this sym matrix (group)."""
    per = out_features if out_per is None else out_per
    return bool(_lib.lib().rwkv_sym_gemm_applies(out_features, in_features, bits, per))


_GEMM_EP = {"store": 0, "add": 1, "relu2_f16": 2}


def rwkvq_gemm_workspace(rows: int, out_features: int, in_features: int) -> int:
    """Bytes of the workspace a long-pass GEMM of this shape splits its K sum
    with (0: the shape runs as one range)."""
    return int(_lib.lib().rwkv_quant_gemm_workspace(rows, out_features, in_features))


def _quant_gemm(entry: str, what: str, x, bufs, out_features: int, in_features: int, code_bits: int, per: int,
                epilogue: str, out: Optional[torch.Tensor], split: bool = True) -> torch.Tensor:
    G = out_features // per
    if x.dim() == 2:
        x = x.unsqueeze(0)
    if x.dim() != 3 or x.shape[0] != G or x.shape[2] != in_features:
        raise ValueError(f"{what} GEMM: input {tuple(x.shape)}, expected [{G}, M, {in_features}]")
    if x.dtype not in (torch.float32, torch.float16):
        x = x.float()
    x = _aligned(x)
    M = x.shape[1]
    ep = _GEMM_EP[epilogue]
    ydt = torch.float16 if ep == 2 else torch.float32
    if out is None:
        if ep == 1:
            raise ValueError(f"{what} GEMM: the add epilogue needs `out`")
        out = torch.empty((M, out_features), dtype=ydt, device=x.device)
    elif out.dtype != ydt or tuple(out.shape) != (M, out_features) or not out.is_contiguous() or \
            out.device != x.device:
        raise ValueError(f"{what} GEMM: out must be a contiguous {ydt} [{M}, {out_features}] tensor on {x.device}")
    need = rwkvq_gemm_workspace(M, out_features, in_features) if split else 0
    ws = torch.empty(need, dtype=torch.uint8, device=x.device) if need else None
    _lib.call(entry, x.data_ptr(), _OUT_DT[x.dtype], M, in_features, M * in_features, *[b.data_ptr() for b in bufs],
              out.data_ptr(), out_features, out_features, in_features, code_bits, per, ep,
              ws.data_ptr() if need else None, need, _stream(x))
    return out


def rwkvq_sb6_gemm(x, qblk, qsqm, ddm, out_features: int, in_features: int, xbits: int = 0,
                   out_per: Optional[int] = None, epilogue: str = "store",
                   out: Optional[torch.Tensor] = None, split: bool = True) -> torch.Tensor:
    """The fp16-base long pass of baseMatmul (X070Backbone.swift:337-356) on
    the matrix cores, straight from the K3 bytes (4, 5 or 6-bit codes): y
    [M, OUT] = fp16(fp16(x)·fp16(W)ᵀ) with fp32 sums.  x [M, IN] (one matrix)
    or [G, M, IN] (G = OUT / out_per row-concatenated matrices, matrix g
    reading x[g]), fp32 or fp16.  epilogue "store" / "add" (fp32 `out`, added
    into) / "relu2_f16" (relu(·)² in an fp16 `out`).  `split`: shapes with few
    output tiles sum K in ranges (a workspace per call; False: one range)."""
    per = out_features if out_per is None else out_per
    if not rwkvq_sb6_gemm_applies(out_features, in_features, xbits, per):
        raise ValueError(f"sb6 GEMM: [{out_features}, {in_features}] xbits={xbits} out_per={per} not taken")
    bufs = _sb6_bufs(qblk, qsqm, ddm, out_features, in_features, xbits)
    return _quant_gemm("rwkv_sb6_gemm", "sb6", x, bufs, out_features, in_features, xbits, per, epilogue, out, split)


def rwkvq_sym_gemm(x, qblk, qs, d, out_features: int, in_features: int, bits: int,
                   out_per: Optional[int] = None, epilogue: str = "store",
                   out: Optional[torch.Tensor] = None, split: bool = True) -> torch.Tensor:
    """rwkvq_sb6_gemm for sym matrices (8-bit codes, or 6-bit in the loader's
    interleave): fp16(W) is exactly rwkvq_dequant_sym's fp16 output (the fp16
    branch of rwkvqDequantSym, RwkvqDequant.swift:350-388)."""
    per = out_features if out_per is None else out_per
    if not rwkvq_sym_gemm_applies(out_features, in_features, bits, per):
        raise ValueError(f"sym GEMM: [{out_features}, {in_features}] bits={bits} out_per={per} not taken")
    bufs = _sym_bufs(qblk, qs, d, out_features, in_features, bits)
    return _quant_gemm("rwkv_sym_gemm", "sym", x, bufs, out_features, in_features, bits, per, epilogue, out, split)


def rwkvq_f16_gemm_applies(rows: int, out_features: int, in_features: int, out_per: Optional[int] = None) -> bool:
    """Whether rwkv_f16_gemm takes this dense fp16 weight (group): OUT and
    out_per multiples of 256, IN of 128."""
    per = out_features if out_per is None else out_per
    return bool(_lib.lib().rwkv_f16_gemm_applies(rows, out_features, in_features, per))


def rwkvq_f16_gemm(x, w, out_per: Optional[int] = None, epilogue: str = "store",
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The fp16 matmul of the long pass on a dense fp16 weight w [OUT, IN]
    (X070Backbone.swift:337-356 after the dequant): y [M, OUT] =
    fp16(x·wᵀ) with fp32 sums, x [M, IN] or [G, M, IN] fp16 (G = OUT /
    out_per, matrix g reading x[g]); epilogues as rwkvq_sb6_gemm.  Bitwise
    the quantised GEMMs' result when w is the fp16 weight they decode."""
    OUT, IN = w.shape
    per = OUT if out_per is None else out_per
    G = OUT // per
    if x.dim() == 2:
        x = x.unsqueeze(0)
    if x.dim() != 3 or x.shape[0] != G or x.shape[2] != IN or x.dtype != torch.float16:
        raise ValueError(f"f16 GEMM: input {tuple(x.shape)} {x.dtype}, expected fp16 [{G}, M, {IN}]")
    if w.dtype != torch.float16:
        raise ValueError(f"f16 GEMM: weight {w.dtype}, expected fp16")
    M = x.shape[1]
    if not rwkvq_f16_gemm_applies(M, OUT, IN, per):
        raise ValueError(f"f16 GEMM: M {M}, [{OUT}, {IN}] out_per={per} not taken")
    x, w = _aligned(x), _aligned(w)
    ep = _GEMM_EP[epilogue]
    ydt = torch.float16 if ep == 2 else torch.float32
    if out is None:
        if ep == 1:
            raise ValueError("f16 GEMM: the add epilogue needs `out`")
        out = torch.empty((M, OUT), dtype=ydt, device=x.device)
    elif out.dtype != ydt or tuple(out.shape) != (M, OUT) or not out.is_contiguous() or out.device != x.device:
        raise ValueError(f"f16 GEMM: out must be a contiguous {ydt} [{M}, {OUT}] tensor on {x.device}")
    _lib.call("rwkv_f16_gemm", x.data_ptr(), M, IN, M * IN, w.data_ptr(), out.data_ptr(), OUT, OUT, IN, per, ep,
              _stream(x))
    return out


def rwkvq_sb6_gemv_batch_applies(rows: int, out_features: int, in_features: int, xbits: int,
                                 out_per: Optional[int] = None) -> bool:
    """Whether the matrix-core batched GEMV takes `rows` input rows of this
    sb6 matrix (group): 4-bit codes, 2..32 rows, matrices of a multiple of 64
    rows."""
    per = out_features if out_per is None else out_per
    return bool(_lib.lib().rwkv_sb6_gemv_batch_applies(rows, out_features, in_features, xbits, per))


def rwkvq_sb6_gemv_batch_prefers(rows: int, out_features: int, in_features: int) -> bool:
    """Where the batched matrix-core GEMV over T16 weights
    (rwkv_sb6_gemv_batch_t16, which picks its own kernel) takes a batch
    instead of the VALU batch kernel.  Up to 4 rows the VALU kernel stays:
    each of its rows is bitwise that row alone (the matrix cores agree to
    fp32 rounding only), at a cost of at most ~1.3 µs per call.  From 5
    rows, where the matrix cores are faster (MI355X, graph-timed per call):
    wherever the entry takes its one-launch row-owned kernel
    (rwkv_sb6_gemv_batch_t16_launches == 1; 768x768 x8 3.5 vs 4.6 µs,
    768x3072 x8 6.5 vs 6.9, 4096x1024 x32 6.4 vs 10.6), 2^24+ weights
    (4096x4096 x8 8.5 vs 12.7), 2^22+ from 8 rows (2048x8192 x8 9.3 vs 15.2)
    and any size from 16 rows (768x3072 x16 8.1 vs 8.5)."""
    n = out_features * in_features
    if rows <= 4:
        return False
    if _lib.lib().rwkv_sb6_gemv_batch_t16_launches(min(rows, 32), out_features, in_features, out_features) == 1:
        return True
    return rows >= 16 or (rows >= 8 and n >= (1 << 22)) or n >= (1 << 24)


_GEMV_EP = {"store": 0, "add": 1, "relu2": 2}


def rwkvq_sb6_gemv_batch(x, qblk, qsqm, ddm, out_features: int, in_features: int, xbits: int = 0,
                         out_per: Optional[int] = None, epilogue: str = "store",
                         out: Optional[torch.Tensor] = None,
                         workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y [N, OUT] = x · Wᵀ for N = 2..32 input rows on the matrix cores, the
    weights streamed once (the batched counterpart of rwkvq_sb6_gemv, within
    fp32 rounding of it per row).  x [N, IN], or [N·K, IN] for K = OUT/out_per
    fused matrices (row o of input n reads x[n·K + o/out_per]).  epilogue
    "store" / "add" (into `out`, the residual stream) / "relu2".  `workspace`:
    an optional uint8 device buffer of rwkv_sb6_gemv_batch_workspace bytes."""
    per = out_features if out_per is None else out_per
    if x.dim() != 2 or x.shape[1] != in_features:
        raise ValueError(f"sb6 batched GEMV: input {tuple(x.shape)}, expected [N, {in_features}]")
    K = out_features // per if per and out_features % per == 0 else 0
    if K == 0 or x.shape[0] % K:
        raise ValueError(f"sb6 batched GEMV: {x.shape[0]} input rows for {out_features} rows of matrices of {per}")
    N = x.shape[0] // K
    if not rwkvq_sb6_gemv_batch_applies(N, out_features, in_features, xbits, per):
        raise ValueError(f"sb6 batched GEMV: N={N} [{out_features}, {in_features}] xbits={xbits} out_per={per} "
                         "not taken")
    x32 = _aligned(x.to(torch.float32))
    qblk, qsqm, ddm = _sb6_bufs(qblk, qsqm, ddm, out_features, in_features, xbits)
    ep = _GEMV_EP[epilogue]
    if out is None:
        if ep == 1:
            raise ValueError("sb6 batched GEMV: the add epilogue needs `out`")
        out = torch.empty((N, out_features), dtype=torch.float32, device=x.device)
    elif out.dtype != torch.float32 or tuple(out.shape) != (N, out_features) or not out.is_contiguous() or \
            out.device != x.device:
        raise ValueError(f"sb6 batched GEMV: out must be a contiguous float32 [{N}, {out_features}] tensor")
    need = int(_lib.lib().rwkv_sb6_gemv_batch_workspace(N, out_features, in_features, per))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    _lib.call("rwkv_sb6_gemv_batch", x32.data_ptr(), N, qblk.data_ptr(), qsqm.data_ptr(), ddm.data_ptr(),
              out.data_ptr(), out_features, in_features, xbits, per, ep, workspace.data_ptr(),
              workspace.numel() * workspace.element_size(), _stream(x32))
    return out


def rwkvq_sb6_t16(qblk, qsqm, ddm, out_features: int, in_features: int):
    """The 4-bit sb6 weights in the matrix cores' T16 order (rwkv_sb6_t16_pack):
    (tq uint8 [OUT·IN/2], ts fp16 [OUT·IN/32], tm bf16 [OUT·IN/16]) on the
    device of qblk, for rwkvq_sb6_gemv_batch_t16."""
    if out_features % 16 or in_features % 256:
        raise ValueError(f"sb6 T16: [{out_features}, {in_features}] (OUT % 16 == 0, IN % 256 == 0)")
    if ddm.dtype in (torch.uint16, torch.int16):   # fp16 bit patterns
        ddm = ddm.view(torch.float16)
    qblk, qsqm, ddm = _sb6_bufs(qblk, qsqm, ddm, out_features, in_features, 0)
    dev = qblk.device
    tq = torch.empty(out_features * in_features // 2, dtype=torch.uint8, device=dev)
    ts = torch.empty(out_features * in_features // 32, dtype=torch.float16, device=dev)
    tm = torch.empty(out_features * in_features // 16, dtype=torch.bfloat16, device=dev)
    _lib.call("rwkv_sb6_t16_pack", qblk.data_ptr(), qsqm.data_ptr(), ddm.data_ptr(), out_features, in_features,
              tq.data_ptr(), ts.data_ptr(), tm.data_ptr(), _stream(qblk))
    return tq, ts, tm


def rwkvq_sb6_gemv_batch_t16(x, tq, ts, tm, out_features: int, in_features: int, out_per: Optional[int] = None,
                             epilogue: str = "store", out: Optional[torch.Tensor] = None,
                             workspace: Optional[torch.Tensor] = None, rows_kernel: bool = False) -> torch.Tensor:
    """rwkvq_sb6_gemv_batch over T16 weights (rwkvq_sb6_t16): the same inputs,
    epilogues and workspace.  `rows_kernel`: the row-owned kernel alone
    (rwkv_sb6_gemv_batch_t16_rows: one launch, no workspace), which the
    default call also picks by itself for matrices of a few thousand rows."""
    per = out_features if out_per is None else out_per
    if x.dim() != 2 or x.shape[1] != in_features:
        raise ValueError(f"sb6 batched GEMV: input {tuple(x.shape)}, expected [N, {in_features}]")
    K = out_features // per if per and out_features % per == 0 else 0
    if K == 0 or x.shape[0] % K:
        raise ValueError(f"sb6 batched GEMV: {x.shape[0]} input rows for {out_features} rows of matrices of {per}")
    N = x.shape[0] // K
    if not rwkvq_sb6_gemv_batch_applies(N, out_features, in_features, 0, per):
        raise ValueError(f"sb6 batched GEMV: N={N} [{out_features}, {in_features}] out_per={per} not taken")
    nw = out_features * in_features
    for t, n, dt in ((tq, nw // 2, torch.uint8), (ts, nw // 32, torch.float16), (tm, nw // 16, torch.bfloat16)):
        if not t.is_cuda or t.dtype != dt or not t.is_contiguous() or t.numel() != n:
            raise ValueError("sb6 batched GEMV: T16 buffers from rwkvq_sb6_t16 expected")
    x32 = _aligned(x.to(torch.float32))
    ep = _GEMV_EP[epilogue]
    if out is None:
        if ep == 1:
            raise ValueError("sb6 batched GEMV: the add epilogue needs `out`")
        out = torch.empty((N, out_features), dtype=torch.float32, device=x.device)
    elif out.dtype != torch.float32 or tuple(out.shape) != (N, out_features) or not out.is_contiguous() or \
            out.device != x.device:
        raise ValueError(f"sb6 batched GEMV: out must be a contiguous float32 [{N}, {out_features}] tensor")
    if rows_kernel:
        _lib.call("rwkv_sb6_gemv_batch_t16_rows", x32.data_ptr(), N, tq.data_ptr(), ts.data_ptr(), tm.data_ptr(),
                  out.data_ptr(), out_features, in_features, per, ep, _stream(x32))
        return out
    need = int(_lib.lib().rwkv_sb6_gemv_batch_workspace(N, out_features, in_features, per))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    _lib.call("rwkv_sb6_gemv_batch_t16", x32.data_ptr(), N, tq.data_ptr(), ts.data_ptr(), tm.data_ptr(),
              out.data_ptr(), out_features, in_features, per, ep, workspace.data_ptr(),
              workspace.numel() * workspace.element_size(), _stream(x32))
    return out


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
        """Read a .rwkvq directly (the reference's RwkvqSidecar.init(rwkvq:only:fusingSym:),
        RwkvqFile.swift:254-492).  The C reader checks the whole manifest
        against the file first (rwkvq_manifest_read); then the buffers of the
        tensors `only` admits are repacked from the mapped file and moved to
        `device`.  A `fusing_sym` group whose members all qualify is read
        straight into one row-concatenated buffer, the members becoming row
        views of it."""
        box = RwkvqContainer(os.path.expanduser(path))
        try:
            man = RwkvqManifest(box, cls.max_format_version)
            admitted = [k for k in man.keys if only is None or only(k)]
            plan = _plan_fused_reads(fusing_sym or {}, man.infos, set(admitted))
            arrays: Dict[str, torch.Tensor] = {}
            fused: Dict[str, RwkvqSymFusedGroup] = {}
            for gid, members in plan.items():
                fused[gid] = _read_sym_group(man, members, arrays, device)
            grouped = {k for members in plan.values() for k in members}
            for key in admitted:
                if key not in grouped:
                    arrays.update(_read_tensor(man, key, device))
            return cls(arrays, man.infos, man.naming, man.n_layer, man.n_embd, man.head_size, man.vocab_size, fused)
        finally:
            box.close()

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
        (the reference's RwkvqSidecar.buildDenseWeights, RwkvqFullConvert.swift:49-140,
        plus `emb.weight` dequantised once as its load(fromSidecar:) does),
        produced by interpreting the name table _X070_BODY: each row maps one
        world key to one x070 key through a shape rule."""
        if not (self.n_layer > 0 and self.n_embd > 0 and self.head_size > 0):
            raise IncompleteManifest("n_layer / n_embd / head_size missing or zero: the manifest does not describe "
                                     "the model")
        if not any(t.kind == RwkvqKind.dense for t in self.tensors.values()):
            raise PartialExport(len(self.tensors))
        D, S = self.n_embd, self.head_size
        out: Dict[str, torch.Tensor] = {}
        for layer in [None] + list(range(self.n_layer)):
            for x070, world, rule in (_X070_GLOBAL if layer is None else _X070_LAYER):
                if layer == 0 and ".tmix.v_" in x070:
                    continue   # layer 0 has no value-residual branch to mix with
                src = world.format(i=layer)
                if src not in self.tensors:
                    raise MissingBuffer(src, "manifest")
                out[x070.format(i=layer)] = _x070_shape(rule, self.dequantize(src, dtype), self.tensors[src], src,
                                                        D, S)
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
        dequantise to `base_dtype` and matmul in it — for an fp16 base and an
        sb6 / sym matrix the matrix-core GEMM does both from the packed bytes
        (the same fp16 weights, products and output rounding).  The reference
        splits the GEMV rows into launches of one (sb6) or four (sym); here all
        rows go in one launch."""
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
        if base_dtype == torch.float16:
            # the fp16 long pass on the matrix cores, from the packed bytes (the
            # input rounded to fp16 here as the kernels would round it, so that
            # shapes with many tiles can take the dense route)
            xin = x2d.to(torch.float16)
            if info.kind == RwkvqKind.sb6 and rwkvq_sb6_gemm_applies(OUT, IN, info.xbits):
                y = rwkvq_sb6_gemm(xin, self._buf(key, "qblk"), self._buf(key, "qsqm"), self._buf(key, "ddm"), OUT,
                                   IN, info.xbits)
                return y.to(x.dtype).reshape(*lead, OUT)
            if info.kind == RwkvqKind.sym and rwkvq_sym_gemm_applies(OUT, IN, info.bits):
                y = rwkvq_sym_gemm(xin, self._buf(key, "qblk"), self._buf(key, "qs"), self._buf(key, "d"), OUT, IN,
                                   info.bits)
                return y.to(x.dtype).reshape(*lead, OUT)
        W = self.dequantize(key, base_dtype)   # the transient dense weight, [OUT, IN]
        if base_dtype == torch.float16 and rwkvq_f16_gemm_applies(rows, OUT, IN):
            return rwkvq_f16_gemm(x2d.to(torch.float16), W).to(x.dtype).reshape(*lead, OUT)
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
        """RwkvqSymGEMV.swift:298-310 on a loaded sidecar: each qualifying sym
        group becomes one row-concatenated buffer, its members row views of it;
        a group that does not qualify is left as separate matrices."""
        return self._fusing(groups, "sym")

    def fusing_sb6(self, groups: Dict[str, List[str]]) -> "RwkvqSidecar":
        """fusing_sym for sb6 groups (an extension: the r/k/v matrices of an
        sb6 model in one launch)."""
        return self._fusing(groups, "sb6")

    def _fusing(self, groups: Dict[str, List[str]], kind: str) -> "RwkvqSidecar":
        arrays = dict(self.arrays)
        made = dict(self.sym_fused if kind == "sym" else self.sb6_fused)
        for gid, keys in groups.items():
            if gid in made:
                continue   # already one buffer: concatenating its views again would copy
            infos = [self.tensors.get(k) for k in keys]
            fields = _loader_fields(RwkvqKind(kind))
            loaded = all(f"{k}::{f}" in arrays for k in keys for f in fields)
            if not loaded or not (_sym_fusable(infos) if kind == "sym" else _sb6_fusable(infos)):
                continue
            OUT = infos[0].out_features
            cat = [torch.cat([arrays[f"{k}::{f}"] for k in keys], 0) for f in fields]
            for i, k in enumerate(keys):
                for f, t in zip(fields, cat):
                    arrays[f"{k}::{f}"] = t[i * OUT:(i + 1) * OUT]
            if kind == "sym":
                made[gid] = RwkvqSymFusedGroup(list(keys), *cat, OUT, infos[0].in_features, infos[0].bits)
            else:
                made[gid] = RwkvqSb6FusedGroup(list(keys), *cat, OUT, infos[0].in_features, infos[0].xbits)
        sym, sb6 = (made, self.sb6_fused) if kind == "sym" else (self.sym_fused, made)
        return RwkvqSidecar(arrays, dict(self.tensors), self.naming, self.n_layer, self.n_embd, self.head_size,
                            self.vocab_size, sym, sb6)

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


def _sb6_fusable(members: List[RwkvqTensorInfo]) -> bool:
    """≥ 2 sb6 matrices of one shape and format that the sb6 GEMV takes."""
    if len(members) < 2 or any(m is None or m.kind != RwkvqKind.sb6 for m in members):
        return False
    m0 = members[0]
    if any(m.shape != m0.shape or m.xbits != m0.xbits or m.super_block != m0.super_block for m in members):
        return False
    return rwkvq_sb6_gemv_applies(m0.out_features, m0.in_features, m0.xbits, m0.super_block, 1)


# x070 names of the dense model body from the world names of a full export
# (the mapping of RwkvqFullConvert.swift:49-140): (x070 key, world key, rule),
# {i} = layer.  Rules: "as_is"; "heads" → [H, S]; "bias" → [D];
# "rank_in" / "rank_out" → the Linear convention A [rank, D] / B [D, rank],
# turned when the manifest marks the tensor `transposed`.
_X070_GLOBAL = (("ln0.weight", "blocks.0.ln0.weight", "as_is"), ("ln0.bias", "blocks.0.ln0.bias", "as_is"),
                ("ln_out.weight", "ln_out.weight", "as_is"), ("ln_out.bias", "ln_out.bias", "as_is"),
                ("emb.weight", "emb.weight", "as_is"))
_X070_LAYER = (
    tuple((f"blocks.{{i}}.{n}.{p}", f"blocks.{{i}}.{n}.{p}", "as_is") for n in ("ln1", "ln2") for p in ("weight", "bias"))
    + tuple((f"blocks.{{i}}.tmix.x_{c}", f"blocks.{{i}}.att.x_{c}", "as_is") for c in "rwkvag")
    + tuple((f"blocks.{{i}}.tmix.{c}", f"blocks.{{i}}.att.{c}", "heads") for c in ("k_k", "k_a", "r_k"))
    + tuple((f"blocks.{{i}}.tmix.{b}_lora_A.weight", f"blocks.{{i}}.att.{b}1", "rank_in") for b in "wagv")
    + tuple((f"blocks.{{i}}.tmix.{b}_lora_B.weight", f"blocks.{{i}}.att.{b}2", "rank_out") for b in "wagv")
    + tuple((f"blocks.{{i}}.tmix.{b}_lora_B.bias", f"blocks.{{i}}.att.{b}0", "bias") for b in "wav")
    + (("blocks.{i}.tmix.ln_x.weight", "blocks.{i}.att.ln_x.weight", "as_is"),
       ("blocks.{i}.tmix.ln_x.bias", "blocks.{i}.att.ln_x.bias", "as_is"),
       ("blocks.{i}.cmix.x_k", "blocks.{i}.ffn.x_k", "as_is")))


def _x070_shape(rule: str, v: torch.Tensor, info: RwkvqTensorInfo, key: str, D: int, S: int) -> torch.Tensor:
    if rule == "as_is":
        return v
    if rule == "heads":
        return v.reshape(D // S, S)
    if rule == "bias":
        return v.reshape(D)
    if info.transposed:
        v = v.t().contiguous()
    side = 1 if rule == "rank_in" else 0
    if v.dim() != 2 or v.shape[side] != D:
        raise ShapeMismatch(key, [-1, D] if side else [D, -1], list(v.shape))
    return v


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
