"""CPU tests of the product's host side: the C ABI library loads and exports
every symbol include/rwkv_hip.h declares; the host-side .rwkvq format work
(unpack6, K3 repack, sym interleave, container, manifest validation,
encoders) against the oracle; the reference's applicability tables.
No device computation happens here."""
import os
import re

import numpy as np
import pytest
import torch

from swiftrwkv_amd import _lib, quant
from tests.test_oracle import make_sb6, make_sym

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "rwkv_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rwkvq?_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = header_symbols()
    assert len(declared) >= 30
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    # and the Python binding knows every one of them
    assert set(declared) <= set(_lib.exported_symbols()) | {"rwkv_get_counters", "rwkv_reset_counters"}
    assert lib.rwkv_abi_version() == 1
    assert lib.rwkv_wkv7_head_size() == 64 and lib.rwkv_wkv7_chunk() == 16


def test_status_strings_and_errors():
    lib = _lib.lib()
    assert [lib.rwkv_status_string(i).decode() for i in range(8)] == \
        ["ok", "shape", "dtype", "unsupported", "format", "hip", "null", "io"]
    # argument validation happens before any device work: a CPU-testable failure path
    st = lib.rwkv_wkv7_seq_fwd(None, None, None, None, None, None, 0, None, None, None, 1, 1, 1, None)
    assert st == 6 and b"non-null" in lib.rwkv_last_error()
    dummy = 8
    st = lib.rwkv_wkv7_train_fwd(*([dummy] * 6), 0, None, dummy, dummy, dummy, dummy, 1, 17, 1, None)
    assert st == 1 and b"multiple of CHUNK" in lib.rwkv_last_error()
    st = lib.rwkv_wkv7_chunk_fwd(*([dummy] * 6), 0, dummy, dummy, dummy, dummy, 1, 15, 1, None)
    assert st == 1
    st = lib.rwkv_wkv7_seq_fwd(*([dummy] * 6), 7, None, dummy, dummy, 1, 1, 1, None)
    assert st == 2
    st = lib.rwkv_wkv7_train_bwd(*([dummy] * 6), 0, None, dummy, dummy, dummy, None, *([dummy] * 6), 0, dummy, 1, 16, 1, 3, None)
    assert st == 3
    st = lib.rwkv_sb6_gemv(dummy, 1, dummy, dummy, dummy, dummy, 16, 200, 0, None)
    assert st == 1
    st = lib.rwkv_sym_gemv(dummy, 1, dummy, dummy, dummy, dummy, 48, 256, 8, 20, None)
    assert st == 1
    st = lib.rwkv_wkv_tail(*([dummy] * 9), 1, 12, 48, 64e-5, None)
    assert st == 1


def test_x070_step_entry_validation():
    """The x070 decode-step entries reject bad arguments before any device work."""
    lib, d = _lib.lib(), 8
    F32, F16 = _lib.F32, _lib.F16
    # layer norm: width not a multiple of 256, or a multiple of 1024 only above 4096; dtype f32/f16
    assert lib.rwkv_layer_norm(d, F32, None, 0, d, d, d, 1, 300, 1e-5, None) == 1
    assert lib.rwkv_layer_norm(d, F32, None, 0, d, d, d, 1, 4608, 1e-5, None) == 1
    assert lib.rwkv_layer_norm(d, _lib.BF16, None, 0, d, d, d, 1, 768, 1e-5, None) == 2
    assert lib.rwkv_layer_norm(d, F32, d, 0, d, d, d, 1, 768, 1e-5, None) == 1      # gather from no rows
    assert lib.rwkv_layer_norm(None, F32, None, 0, None, None, None, 0, 768, 1e-5, None) == 0   # N = 0
    # shift + lerps: 1 or 6 coefficients, out1 needed for 6
    assert lib.rwkv_x070_shift_mix(d, d, d, d, d, 3, d, d, 1, 768, 1e-5, None) == 1
    assert lib.rwkv_x070_shift_mix(d, d, d, d, d, 6, d, None, 1, 768, 1e-5, None) == 6
    # low-rank: ranks multiples of 8, matrices f16/f32
    assert lib.rwkv_x070_lora_in(d, d, F16, 60, 64, 32, 128, 1, d, 1, 768, None) == 1
    assert lib.rwkv_x070_lora_in(d, d, _lib.BF16, 64, 64, 32, 128, 1, d, 1, 768, None) == 2
    # tmix core: v branch buffers needed above layer 0
    args = [d] * 6 + [F16, 64, 64, 32, 128] + [d, d, None] + [d] * 5 + [d, 0, d, d, 1, 12, 64e-5, None, None, None]
    assert lib.rwkv_x070_tmix_core(*args) == 6
    args = [d] * 6 + [F16, 64, 64, 32, 128] + [d, d, d] + [d] * 5 + [d, 0, d, d, 1, 12, 64e-5, d, None, None]
    assert lib.rwkv_x070_tmix_core(*args) == 6                                                    # shift copy: both
    # launches forming their GEMV inputs: the x070 plans, batch 1, 4-bit
    assert lib.rwkv_x070_ln_fused_applies(768, 3072, 0) == 1
    assert lib.rwkv_x070_ln_fused_applies(2048, 8192, 0) == 1
    assert lib.rwkv_x070_ln_fused_applies(4096, 14336, 0) == 0                                    # grids > one round
    assert lib.rwkv_x070_ln_fused_applies(768, 3072, 1) == 0
    assert lib.rwkv_x070_ln_fused_applies(8192, 32768, 0) == 0                                     # D > 4096
    assert lib.rwkv_x070_ffn_value(d, d, d, d, d, 768, 3072, 0, d, None, None) == 6              # copy: both
    assert lib.rwkv_x070_ffn_key_ln(d, d, d, None, d, 1e-5, d, d, d, d, d, 3072, 768, 0, None) == 6
    assert lib.rwkv_x070_rkv_lora_ln(*([d] * 5), 1e-5, d, d, d, d, d, 768, 0, d, _lib.BF16, 64, 64, 32, 128, 1, d,
                                     None) == 2                                                    # fp16 matrices
    # r/k/v GEMV + low-rank first layers in one launch: the checks of both entries
    rkl = lambda *a: lib.rwkv_x070_rkv_lora(d, d, d, d, d, *a)
    assert rkl(3 * 768, 768, 0, 768, None, d, F16, 64, 64, 32, 128, 1, d, None) == 6            # no xmix
    assert rkl(3 * 768, 768, 0, 768, d, d, _lib.BF16, 64, 64, 32, 128, 1, d, None) == 2         # matrix dtype
    assert rkl(3 * 768, 768, 0, 768, d, d, F16, 60, 64, 32, 128, 1, d, None) == 1               # ranks
    assert rkl(3 * 768, 768, 0, 700, d, d, F16, 64, 64, 32, 128, 1, d, None) == 1               # out_per
    assert rkl(3 * 768, 768, 3, 768, d, d, F16, 64, 64, 32, 128, 1, d, None) == 1               # xbits
    # GEMV epilogue code
    assert lib.rwkv_sb6_gemv_ep(d, 1, d, d, d, d, 256, 256, 0, 3, None) == 1
    assert lib.rwkv_sym_gemv_ep(d, 1, d, d, d, d, 256, 256, 8, -1, None) == 1


def test_applies_tables_are_the_reference_ones():
    # RwkvqSb6GEMVTests.swift:80-100
    assert quant.rwkvq_sb6_gemv_config(65536, 2048, 0) == (4, 4)
    assert quant.rwkvq_sb6_gemv_config(8192, 2048, 0) == (2, 2)
    assert quant.rwkvq_sb6_gemv_config(8192, 2048, 1) == (4, 4)
    assert quant.rwkvq_sb6_gemv_config(2048, 8192, 0) == (4, 4)
    assert not quant.rwkvq_sb6_gemv_applies(24, 256, 0, 8, 1)
    assert not quant.rwkvq_sb6_gemv_applies(16, 96, 0, 8, 1)
    assert not quant.rwkvq_sb6_gemv_applies(16, 256, 0, 4, 1)
    assert not quant.rwkvq_sb6_gemv_applies(768, 768, 0, 8, 2)
    assert quant.rwkvq_sb6_gemv_applies(768, 768, 0, 8, 1)
    assert quant.rwkvq_sb6_gemv_applies(8196, 768, 0, 8, 1)       # (2,2) ⇒ OUT % 4
    assert not quant.rwkvq_sb6_gemv_applies(8196, 768, 1, 8, 1)   # (4,4) ⇒ OUT % 16
    # RwkvqSymGEMVTests.swift:75-86
    assert not quant.rwkvq_sym_gemv_applies(24, 256, 8, 1)
    assert not quant.rwkvq_sym_gemv_applies(16, 48, 8, 1)
    assert quant.rwkvq_sym_gemv_applies(16, 256, 6, 4)
    assert not quant.rwkvq_sym_gemv_applies(16, 256, 6, 5)
    assert quant.RWKVQ_SYM_GEMV_MAX_ROWS == 4
    from swiftrwkv_amd import kernel
    assert kernel.wkv_tail_applies(64) and not kernel.wkv_tail_applies(48)
    # X070Backbone.defaultShortPassRows: max(4, D / 128) sym, max(4, D / 256) sb6
    assert quant.default_short_pass_rows(768, sym=False) == 4
    assert quant.default_short_pass_rows(2048, sym=False) == 8
    assert quant.default_short_pass_rows(2048, sym=True) == 16
    assert quant.default_short_pass_rows(4096, sym=True) == 32


def test_unpack6_product_equals_oracle(orc):
    rng = np.random.default_rng(0)
    b = rng.integers(0, 256, (4096, 6), dtype=np.uint8)
    assert np.array_equal(quant.rwkvq_unpack6x8(b), orc.unpack6x8(b))


@pytest.mark.parametrize("xbits", [0, 1, 2])
def test_sb6_to_k3_product_equals_oracle(orc, xbits):
    rng = np.random.default_rng(xbits)
    OUT, IN = 7, 512
    t = make_sb6(OUT, IN, xbits, rng)
    got = quant.rwkvq_sb6_to_k3(t["cp"], t["qsqm_disk"], t["d"], t["dm"], t["qh"], t["qh2"], (OUT, IN))
    want = orc.sb6_to_k3(t["cp"], t["qh"], t["qh2"], t["qsqm_disk"], t["d"].view(np.uint16),
                         t["dm"].view(np.uint16), OUT, IN)
    for g, w in zip(got, want):
        assert np.array_equal(np.asarray(g), np.asarray(w))


def test_sym_interleave_product_equals_oracle(orc):
    rng = np.random.default_rng(5)
    t = make_sym(9, 768, 6, rng)
    assert np.array_equal(quant.rwkvq_sym_interleave(t["cp"], t["qh"], t["qh2"], (9, 768)),
                          orc.sym_interleave(t["cp"], t["qh"], t["qh2"], 9, 768))


@pytest.mark.parametrize("bits", [4, 5, 6])
def test_sb6_encoder_round_trip(orc, bits):
    """Encoder (parity unpinned: not in the reference) — range and error invariants."""
    rng = np.random.default_rng(bits)
    OUT, IN = 32, 768
    w = (rng.standard_normal((OUT, IN)) * 0.02).astype(np.float32)
    disk = quant.encode_sb6(w, bits)
    assert disk["gw_qsqm"].shape == (OUT, IN // 256, 12)
    qblk, qsqm, ddm, xb = quant.rwkvq_sb6_to_k3(disk["codes_packed"], disk["gw_qsqm"], disk["gw_d"], disk["gw_dm"],
                                                disk.get("gw_qh"), disk.get("gw_qh2"), (OUT, IN))
    assert xb == bits - 4
    deq = orc.sb6_dequant(qblk, qsqm, ddm, OUT, IN, xb)
    step = (w.reshape(OUT, -1, 32).max(-1) - w.reshape(OUT, -1, 32).min(-1)) / ((1 << bits) - 1)
    err = np.abs(deq - w).reshape(OUT, -1, 32).max(-1)
    # half a quantisation step plus the 6-bit scale / min rounding
    assert np.all(err <= 0.5 * step + 0.04 * np.abs(w).reshape(OUT, -1, 32).max(-1) + 1e-6)
    rel = np.linalg.norm(deq - w) / np.linalg.norm(w)
    assert rel < {4: 0.12, 5: 0.06, 6: 0.035}[bits]


@pytest.mark.parametrize("bits", [8, 6])
def test_sym_encoder_round_trip(orc, bits):
    rng = np.random.default_rng(bits)
    OUT, IN = 16, 512
    w = (rng.standard_normal((OUT, IN)) * 0.02).astype(np.float32)
    disk = quant.encode_sym(w, bits)
    qblk = disk["codes"].view(np.uint8) if bits == 8 else quant.rwkvq_sym_interleave(
        disk["codes_packed"], disk["gw_qh"], disk["gw_qh2"], (OUT, IN))
    deq = orc.sym_dequant(qblk, disk["gw_qs"].view(np.uint8), disk["gw_d"].view(np.uint16), OUT, IN, bits)
    rel = np.linalg.norm(deq - w) / np.linalg.norm(w)
    assert rel < {8: 0.01, 6: 0.04}[bits]


# ───────────────────────────── container / manifest ─────────────────────────────

def _small_file(path, kinds=("sb6",)):
    rng = np.random.default_rng(0)
    tensors = {}
    for i, kind in enumerate(kinds):
        w = (rng.standard_normal((32, 512)) * 0.02).astype(np.float32)
        tensors[f"blocks.{i}.att.key.weight"] = quant.sb6_entry(w, 5) if kind == "sb6" else quant.sym_entry(w, 6)
    quant.write_rwkvq(path, tensors, n_layer=len(kinds), n_embd=512, vocab_size=64)
    return tensors


def test_container_round_trip_and_host_load(tmp_path, orc):
    p = str(tmp_path / "m.rwkvq")
    tensors = _small_file(p, ("sb6", "sym"))
    box = quant.RwkvqContainer(p)
    assert "blocks.0.att.key.weight::gw_qsqm" in box.names
    assert box.shape("blocks.0.att.key.weight::gw_qsqm") == (32, 2, 12)
    assert box.dtype("blocks.0.att.key.weight::gw_d") == "F16"
    assert np.array_equal(box.array("blocks.1.att.key.weight::gw_qs"), tensors["blocks.1.att.key.weight"][1]["gw_qs"])
    box.close()
    sc = quant.RwkvqSidecar.from_rwkvq(p, device="cpu")
    assert sc.n_layer == 2 and sc.n_embd == 512 and sc.naming == "world"
    info = sc.tensors["blocks.0.att.key.weight"]
    assert info.kind == quant.RwkvqKind.sb6 and info.xbits == 1 and info.bits == 5 and info.is_quantized_base
    assert sc.tensors["blocks.1.att.key.weight"].bits == 6
    # buffers in loader layout, equal to the oracle repack of the disk buffers
    disk = tensors["blocks.0.att.key.weight"][1]
    want = orc.sb6_to_k3(disk["codes_packed"], disk["gw_qh"], None, disk["gw_qsqm"], disk["gw_d"].view(np.uint16),
                         disk["gw_dm"].view(np.uint16), 32, 512)
    assert np.array_equal(sc.arrays["blocks.0.att.key.weight::qblk"].numpy(), want[0])
    assert np.array_equal(sc.arrays["blocks.0.att.key.weight::qsqm"].numpy(), want[1])
    assert np.array_equal(sc.arrays["blocks.0.att.key.weight::ddm"].view(torch.int16).numpy().view(np.uint16), want[2])
    # partial load: manifest validated in full, buffers only for the wanted tensor
    part = quant.RwkvqSidecar.from_rwkvq(p, only=lambda k: k.startswith("blocks.1"), device="cpu")
    assert part.contains("blocks.0.att.key.weight")
    with pytest.raises(quant.MissingBuffer):
        part.dequantize("blocks.0.att.key.weight")


def test_container_rejects_foreign_files(tmp_path):
    # RwkvqFileTests.swift:129-156
    zipf = tmp_path / "old.rwkvq"
    zipf.write_bytes(bytes([0x50, 0x4B, 0x03, 0x04]) + bytes(64))
    with pytest.raises(quant.MalformedManifest, match="pickle"):
        quant.RwkvqSidecar.from_rwkvq(str(zipf), device="cpu")
    plain = tmp_path / "plain.safetensors"
    quant.write_safetensors(str(plain), {"x": np.float32([1, 2, 3])})
    with pytest.raises(quant.MalformedManifest, match="not an .rwkvq file"):
        quant.RwkvqSidecar.from_rwkvq(str(plain), device="cpu")
    good = tmp_path / "good.rwkvq"
    _small_file(str(good))
    cut = tmp_path / "cut.rwkvq"
    cut.write_bytes(good.read_bytes()[:3000])
    with pytest.raises(quant.MalformedManifest):
        quant.RwkvqSidecar.from_rwkvq(str(cut), device="cpu")
    with pytest.raises(quant.MissingFile):
        quant.RwkvqSidecar.from_rwkvq(str(tmp_path / "no.rwkvq"), device="cpu")
    short = tmp_path / "short.rwkvq"
    short.write_bytes(b"\x01\x02")
    with pytest.raises(quant.MalformedManifest):
        quant.RwkvqContainer(str(short))
    # header length beyond the file, unknown dtype, offsets that disagree with the shape
    bad = tmp_path / "bad.rwkvq"
    bad.write_bytes((10 ** 6).to_bytes(8, "little") + b"{}")
    with pytest.raises(quant.MalformedManifest, match="outside the file"):
        quant.RwkvqContainer(str(bad))
    big = 2 ** 63
    for hdr in (b'{"x":{"dtype":"Q7","shape":[1],"data_offsets":[0,1]}}',
                b'{"x":{"dtype":"F32","shape":[2],"data_offsets":[0,4]}}',
                # offsets whose sum with the header end wraps past 2^63
                b'{"x":{"dtype":"U8","shape":[8],"data_offsets":[%d,%d]}}' % (big - 11, big - 3),
                # a shape whose byte size wraps int64
                b'{"x":{"dtype":"F32","shape":[%d,4],"data_offsets":[0,0]}}' % (2 ** 62),
                # an integer beyond int64
                b'{"x":{"dtype":"U8","shape":[8],"data_offsets":[0,%d]}}' % (2 ** 70)):
        f = tmp_path / "hdr.rwkvq"
        f.write_bytes(len(hdr).to_bytes(8, "little") + hdr + bytes(8))
        with pytest.raises(quant.MalformedManifest):
            quant.RwkvqContainer(str(f))


def test_manifest_validation_errors(tmp_path):
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((16, 512)) * 0.02).astype(np.float32)
    m, bufs = quant.sb6_entry(w, 4)

    def write(entry, buffers, **kw):
        p = str(tmp_path / "v.rwkvq")
        quant.write_rwkvq(p, {"k.weight": (entry, buffers)}, **kw)
        return p

    with pytest.raises(quant.MalformedManifest, match="blocks of 32 columns"):
        quant.RwkvqSidecar.from_rwkvq(write(dict(m, gw_gs=64), bufs), device="cpu")
    with pytest.raises(quant.MalformedManifest, match="bit planes"):
        quant.RwkvqSidecar.from_rwkvq(write(dict(m, bits=5), bufs), device="cpu")
    with pytest.raises(quant.ShapeMismatch):
        quant.RwkvqSidecar.from_rwkvq(write(m, dict(bufs, gw_qsqm=bufs["gw_qsqm"].reshape(16, 24))), device="cpu")
    with pytest.raises(quant.MissingBuffer):
        quant.RwkvqSidecar.from_rwkvq(write(m, {k: v for k, v in bufs.items() if k != "gw_dm"}), device="cpu")
    with pytest.raises(quant.MalformedManifest, match="n_blocks"):
        quant.RwkvqSidecar.from_rwkvq(write(dict(m, n_blocks=3), bufs), device="cpu")
    with pytest.raises(quant.MalformedManifest, match="format_version"):
        quant.RwkvqSidecar.from_rwkvq(write(m, bufs, format_version=3), device="cpu")
    with pytest.raises(quant.MalformedManifest, match="unknown layout"):
        quant.RwkvqSidecar.from_rwkvq(write(dict(m, kind="q9"), bufs), device="cpu")
    sm, sbufs = quant.sym_entry(w, 8)
    with pytest.raises(quant.MalformedManifest, match="codes buffer"):
        quant.RwkvqSidecar.from_rwkvq(write(dict(sm, bits=6), sbufs), device="cpu")


@pytest.mark.parametrize("bits", [4, 5, 6])
def test_short_sb6_buffers_are_rejected(tmp_path, bits):
    """Every buffer an sb6 decode reads must be complete: a truncated one is a
    ShapeMismatch naming it, before any repack could read past it."""
    w = (np.random.default_rng(2).standard_normal((16, 512)) * 0.02).astype(np.float32)
    m, bufs = quant.sb6_entry(w, bits)
    p = str(tmp_path / "s.rwkvq")
    for field in bufs:
        short = dict(bufs, **{field: bufs[field].reshape(-1)[:-1]})
        quant.write_rwkvq(p, {"k.weight": (m, short)})
        with pytest.raises(quant.ShapeMismatch) as e:
            quant.RwkvqSidecar.from_rwkvq(p, device="cpu")
        assert e.value.tensor == "k.weight" and field in str(e.value), field
    if bits == 6:   # a second high-bit plane without the first
        quant.write_rwkvq(p, {"k.weight": (dict(m, bits=5), {f: v for f, v in bufs.items() if f != "gw_qh"})})
        with pytest.raises(quant.MalformedManifest, match="gw_qh2"):
            quant.RwkvqSidecar.from_rwkvq(p, device="cpu")


@pytest.mark.parametrize("bits", [8, 6])
def test_short_sym_buffers_are_rejected(tmp_path, bits):
    w = (np.random.default_rng(3).standard_normal((16, 512)) * 0.02).astype(np.float32)
    m, bufs = quant.sym_entry(w, bits)
    p = str(tmp_path / "s.rwkvq")
    for field in bufs:
        short = dict(bufs, **{field: bufs[field].reshape(-1)[:-1]})
        quant.write_rwkvq(p, {"k.weight": (m, short)})
        with pytest.raises(quant.ShapeMismatch) as e:
            quant.RwkvqSidecar.from_rwkvq(p, device="cpu")
        assert field in str(e.value), field
    # a scale table that is the right size but not [OUT, IN/256]
    quant.write_rwkvq(p, {"k.weight": (m, dict(bufs, gw_d=bufs["gw_d"].reshape(32, 1)))})
    with pytest.raises(quant.ShapeMismatch, match="gw_d"):
        quant.RwkvqSidecar.from_rwkvq(p, device="cpu")


def test_repack_wrappers_check_buffer_sizes():
    w = (np.random.default_rng(5).standard_normal((8, 256)) * 0.02).astype(np.float32)
    d = quant.encode_sb6(w, 5)
    args = [d["codes_packed"], d["gw_qsqm"], d["gw_d"], d["gw_dm"], d["gw_qh"], None]
    quant.rwkvq_sb6_to_k3(*args, (8, 256))
    for i in range(5):
        bad = list(args)
        bad[i] = bad[i].reshape(-1)[:-1]
        with pytest.raises(ValueError):
            quant.rwkvq_sb6_to_k3(*bad, (8, 256))
    s6 = quant.encode_sym(w, 6)
    quant.rwkvq_sym_interleave(s6["codes_packed"], s6["gw_qh"], s6["gw_qh2"], (8, 256))
    with pytest.raises(ValueError):
        quant.rwkvq_sym_interleave(s6["codes_packed"][:-1], s6["gw_qh"], s6["gw_qh2"], (8, 256))


def test_manifest_transposed_default_follows_world_naming(tmp_path):
    """The reader's default for `transposed` is the world naming rule
    (RwkvqFileTests.swift:123-127) unless the manifest says otherwise."""
    keys = ["blocks.1.att.w1", "blocks.1.att.g2", "blocks.1.att.w0", "blocks.1.ffn.key.weight", "x.att.a1"]
    ent = lambda: ({"kind": "dense", "shape": [4]}, {"dense": np.ones(4, np.float16)})
    p = str(tmp_path / "n.rwkvq")
    quant.write_rwkvq(p, {k: ent() for k in keys} | {"blocks.2.att.v1": ({"kind": "dense", "shape": [4],
                                                                           "transposed": False},
                                                                          {"dense": np.ones(4, np.float16)})})
    sc = quant.RwkvqSidecar.from_rwkvq(p, device="cpu")
    for k in keys:
        assert sc.tensors[k].transposed == quant.is_raw_lora_world(k), k
    assert not sc.tensors["blocks.2.att.v1"].transposed
    quant.write_rwkvq(p, {k: ent() for k in keys}, naming="x070")
    assert not any(t.transposed for t in quant.RwkvqSidecar.from_rwkvq(p, device="cpu").tensors.values())


def test_sym_group_read_at_load_equals_fusing_after(tmp_path):
    """A fusing_sym group read straight into one buffer holds the same bytes
    as the members loaded alone and concatenated afterwards; members are row
    views of it; a group with a non-sym member is not fused."""
    rng = np.random.default_rng(4)
    T = {f"blocks.0.att.{m}.weight": quant.sym_entry((rng.standard_normal((32, 256)) * 0.02).astype(np.float32), 6)
         for m in ("receptance", "key", "value")}
    T["blocks.0.att.output.weight"] = quant.sb6_entry((rng.standard_normal((32, 256)) * 0.02).astype(np.float32), 4)
    p = str(tmp_path / "g.rwkvq")
    quant.write_rwkvq(p, T)
    rkv = [f"blocks.0.att.{m}.weight" for m in ("receptance", "key", "value")]
    groups = {"att0": rkv, "mixed": ["blocks.0.att.output.weight", rkv[0]]}
    at_load = quant.RwkvqSidecar.from_rwkvq(p, fusing_sym=groups, device="cpu")
    after = quant.RwkvqSidecar.from_rwkvq(p, device="cpu").fusing_sym(groups)
    assert set(at_load.sym_fused) == set(after.sym_fused) == {"att0"}
    for f in ("qblk", "qs", "d"):
        a, b = getattr(at_load.sym_fused["att0"], f), getattr(after.sym_fused["att0"], f)
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), f
        for i, k in enumerate(rkv):
            v = at_load.arrays[f"{k}::{f}"]
            assert v.untyped_storage().data_ptr() == a.untyped_storage().data_ptr(), (k, f)
            assert torch.equal(v.view(torch.uint8), a[i * 32:(i + 1) * 32].view(torch.uint8)), (k, f)


def test_lora_orientation_naming_rule():
    # RwkvqFileTests.swift:123-127
    assert quant.is_raw_lora_world("blocks.11.att.g2")
    assert quant.is_raw_lora_world("blocks.0.att.w1")
    assert not quant.is_raw_lora_world("blocks.0.att.w0")
    assert not quant.is_raw_lora_world("blocks.0.att.key.weight")
    assert not quant.is_raw_lora_world("blocks.0.ffn.w1")


def test_batched_gemv_kernel_choice_rules():
    """The T16 batched GEMV's one-launch row-owned kernel: up to 2^24 weights
    for K <= 3072, and for K <= 4096 where its grid is up to 64 workgroups or
    more than 256 (row-tile pairs); K slices plus their reduction (two
    launches) elsewhere; 0 where the batched GEMV does not apply.  The
    decoder's preference for it keeps batches of up to 4 rows on the VALU
    kernel (bitwise each row alone)."""
    from swiftrwkv_amd import _lib
    L = _lib.lib()
    launches = lambda N, OUT, IN, per=None: int(L.rwkv_sb6_gemv_batch_t16_launches(N, OUT, IN, per or OUT))
    assert launches(32, 1024, 1024) == 1
    assert launches(32, 16384, 1024) == 1           # 2^24 weights
    assert launches(32, 32768, 768) == 2 and launches(8, 65536, 768) == 2
    assert launches(16, 8192, 2048) == 1 and launches(16, 16384, 2048) == 2
    assert launches(16, 3072, 3072) == 1
    assert launches(8, 1024, 4096) == 1 and launches(16, 1024, 4096) == 1   # 64 workgroups
    assert launches(17, 1024, 4096) == 2 and launches(16, 4096, 4096) == 2  # 128, 256
    assert launches(32, 4096, 4096) == 1            # 512: pairs of row tiles
    assert launches(16, 12288, 4096) == 2 and launches(16, 2048, 8192) == 2
    assert launches(8, 3 * 768, 768, 768) == 1      # fused r/k/v group
    assert launches(1, 768, 768) == 0 and launches(33, 768, 768) == 0 and launches(8, 768, 800) == 0
    pref = quant.rwkvq_sb6_gemv_batch_prefers
    assert not pref(4, 768, 768) and pref(5, 768, 768)
    assert not pref(4, 4096, 4096) and pref(8, 4096, 4096)
    assert not pref(8, 256, 8192) and pref(16, 256, 8192)   # 2^21 weights, K past the row-owned kernel


def test_x070_launch_count():
    """launches_per_token over mixed projection kinds: a fused sb6 / sym GEMV
    is one launch, a dense projection its GEMM plus epilogue kernels (store or
    residual add: 1; relu²: 3), unfused r / k / v at N > 1 two staging copies
    per matrix."""
    from swiftrwkv_amd.x070 import Proj, X070Decoder
    d = X070Decoder.__new__(X070Decoder)
    d.L = 2
    d.fuse_rkv_lora = False
    d.fuse_ln = False
    P = lambda kind: Proj(kind, (), 64, 64)
    d.proj = {"blocks.0.att.rkv": P("sb6"), "blocks.1.att.rkv": [P("sym"), P("sb6"), P("dense")],
              "head.weight": P("dense")}
    for l in range(2):
        for k in ("att.output", "ffn.key", "ffn.value"):
            d.proj[f"blocks.{l}.{k}.weight"] = P("sb6")
    d.proj["blocks.0.ffn.key.weight"] = P("dense")
    # layer 0: 4 + 1 + (1 + 4 + 1); layer 1: 4 + (1 + 1 + 2) + 3; ln / head: 2 + 2
    assert d.launches_per_token(1) == 11 + 11 + 4
    assert d.launches_per_token(2) == 11 + 11 + 6 + 4
    for k in list(d.proj):
        d.proj[k] = P("sb6")
    assert d.launches_per_token(1) == 8 * 2 + 3
    # batch 1, a fused 4-bit sb6 r/k/v group and fp16 low-rank matrices: the
    # group and lora_in share one launch
    d.fuse_rkv_lora = True
    d.layers = [{"wcat": torch.empty(0, dtype=torch.float16)}] * 2
    for l in range(2):
        d.proj[f"blocks.{l}.att.rkv"] = Proj("sb6", (), 192, 64, out_per=64)
    assert d.launches_per_token(1) == 7 * 2 + 3
    # and forming the rows: r/k/v + low-rank, tmix core, o, ffn key, ffn value
    d.fuse_ln, d.D, d.F = True, 768, 3072
    assert d.launches_per_token(1) == 5 * 2 + 3
    assert d.launches_per_token(2) == 8 * 2 + 3   # batches keep the shift_mix launches
    assert d.launches_per_token(2) == 8 * 2 + 3
    d.layers = [{"wcat": torch.empty(0, dtype=torch.float32)}] * 2
    assert d.launches_per_token(1) == 8 * 2 + 3
