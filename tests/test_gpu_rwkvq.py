"""GPU parity of the .rwkvq dequant and GEMV kernels.

Dequant: bit-exact against the oracle (pure functions of bytes), all layouts
and storage types (RwkvqFileTests, RwkvqDTypeTests).  GEMV: ≤ 2e-5 relative
to an fp64 matmul with the dequantised weights (the reference's own bound,
RwkvqSb6GEMVTests.swift:53-77), bit-exact on one-hot inputs, fused ==
separate bitwise (RwkvqSymGEMVTests.swift:164-201).
"""
import json
import os
import sys

import numpy as np
import pytest
import torch

from swiftrwkv_amd import _lib, quant as Q
from tests.test_oracle import GOLD, make_sb6, make_sym

pytestmark = pytest.mark.gpu
DEV = "cuda"
GEMV_TOL = 2e-5


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def rel(ref, got):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(ref - np.asarray(got, np.float64)).max() / (np.abs(ref).max() + 1e-30))


def sb6_tensor(orc, OUT, IN, xbits, seed, degenerate=False):
    rng = np.random.default_rng(seed)
    t = make_sb6(OUT, IN, xbits, rng, degenerate)
    qblk, qsqm, ddm, xb = orc.sb6_to_k3(t["cp"], t["qh"], t["qh2"], t["qsqm_disk"], t["d"].view(np.uint16),
                                        t["dm"].view(np.uint16), OUT, IN)
    return qblk, qsqm, ddm.view(np.float16)


def sym_tensor(orc, OUT, IN, bits, seed):
    rng = np.random.default_rng(seed)
    t = make_sym(OUT, IN, bits, rng)
    qblk = t["qblk"] if bits == 8 else orc.sym_interleave(t["cp"], t["qh"], t["qh2"], OUT, IN)
    return qblk, t["qs"].view(np.uint8), t["d"]


DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def as_bits(t: torch.Tensor):
    if t.dtype == torch.float32:
        return t.cpu().numpy()
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("xbits", [0, 1, 2])
def test_sb6_dequant_bit_exact(orc, xbits):
    OUT, IN = 48, 768
    case(f"sb6 dequant xbits={xbits}")
    qblk, qsqm, ddm = sb6_tensor(orc, OUT, IN, xbits, seed=xbits, degenerate=True)
    for name, dt in DT.items():
        got = Q.rwkvq_dequant_dense(dev(qblk), dev(qsqm), dev(ddm), OUT, IN, 8, xbits, dt)
        want = orc.sb6_dequant(qblk, qsqm, ddm.view(np.uint16), OUT, IN, xbits, name)
        assert got.dtype == dt and np.array_equal(as_bits(got).view(want.dtype), want), name


@pytest.mark.parametrize("bits", [8, 6])
def test_sym_dequant_bit_exact(orc, bits):
    OUT, IN = 40, 1024
    case(f"sym dequant bits={bits}")
    qblk, qs, d = sym_tensor(orc, OUT, IN, bits, seed=bits)
    for name, dt in DT.items():
        got = Q.rwkvq_dequant_sym(dev(qblk), dev(qs), dev(d), OUT, IN, bits, dt)
        want = orc.sym_dequant(qblk, qs, d.view(np.uint16), OUT, IN, bits, name)
        assert np.array_equal(as_bits(got).view(want.dtype), want), name


def test_sym_off_superblock_known_answer():
    case("sym KAT IN=48 (RwkvqFileTests.swift:237-256)")
    kat = json.load(open(os.path.join(GOLD, "sym8_kat.json")))
    got = Q.rwkvq_dequant_sym(dev(np.array(kat["codes_u8"], np.uint8).reshape(2, 48)),
                              dev(np.array(kat["qs_u8"], np.uint8).reshape(2, 3)),
                              dev(np.array(kat["d_f16_bits"], np.uint16).view(np.float16).reshape(2, 1)),
                              2, 48, 8, torch.float32)
    assert np.array_equal(got.cpu().numpy().reshape(-1), np.array(kat["expected_f32"], np.float32))


# 32 x 7168: 224 column units per row, 7 per lane (several passes, inputs read from global memory)
GEMV_SHAPES = [(768, 768), (3072, 768), (768, 3072), (2048, 2048), (24, 256), (32, 7168)]


@pytest.mark.parametrize("xbits", [0, 1, 2])
@pytest.mark.parametrize("OUT,IN", GEMV_SHAPES)
def test_sb6_gemv_matches_fp64(orc, xbits, OUT, IN):
    case(f"sb6 gemv {OUT}x{IN} xbits={xbits}")
    qblk, qsqm, ddm = sb6_tensor(orc, OUT, IN, xbits, seed=OUT + IN + xbits)
    rng = np.random.default_rng(17)
    for N in (1, 3, 6):
        x = rng.standard_normal((N, IN)).astype(np.float32)
        y = Q.rwkvq_sb6_gemv(dev(x), dev(qblk), dev(qsqm), dev(ddm), OUT, IN, xbits)
        want = orc.sb6_gemv_f64(x, qblk, qsqm, ddm.view(np.uint16), OUT, IN, xbits)
        assert y.shape == (N, OUT)
        assert rel(want, y.cpu().numpy()) < GEMV_TOL, N


def test_sb6_gemv_head_shape(orc):
    OUT, IN = 65536, 768
    case("sb6 gemv head 65536x768")
    qblk, qsqm, ddm = sb6_tensor(orc, OUT, IN, 0, seed=99)
    x = np.random.default_rng(1).standard_normal((1, IN)).astype(np.float32)
    y = Q.rwkvq_sb6_gemv(dev(x), dev(qblk), dev(qsqm), dev(ddm), OUT, IN, 0)
    want = orc.sb6_gemv_f64(x, qblk, qsqm, ddm.view(np.uint16), OUT, IN, 0)
    assert rel(want, y.cpu().numpy()) < GEMV_TOL


def test_gemv_one_hot_is_bit_exact_dequant_column(orc):
    case("one-hot GEMV == dequant column")
    OUT, IN = 512, 768
    cols = [0, 31, 32, 400, 767]
    x = np.zeros((len(cols), IN), np.float32)
    x[np.arange(len(cols)), cols] = 1.0
    for xb in (2, 0):   # 6-bit and 4-bit codes
        qblk, qsqm, ddm = sb6_tensor(orc, OUT, IN, xb, seed=5, degenerate=True)
        W = orc.sb6_dequant(qblk, qsqm, ddm.view(np.uint16), OUT, IN, xb)
        y = Q.rwkvq_sb6_gemv(dev(x), dev(qblk), dev(qsqm), dev(ddm), OUT, IN, xb).cpu().numpy()
        assert np.array_equal(y, W[:, cols].T), xb
        # a power-of-two input scale is exact as well
        y4 = Q.rwkvq_sb6_gemv(dev(x * 0.25), dev(qblk), dev(qsqm), dev(ddm), OUT, IN, xb).cpu().numpy()
        assert np.array_equal(y4, (W[:, cols] * np.float32(0.25)).T), xb
    for bits in (8, 6):
        sq, qs, d = sym_tensor(orc, OUT, IN, bits, seed=bits)
        Ws = orc.sym_dequant(sq, qs, d.view(np.uint16), OUT, IN, bits)
        ys = Q.rwkvq_sym_gemv(dev(x), dev(sq), dev(qs), dev(d), OUT, IN, bits).cpu().numpy()
        assert np.array_equal(ys, Ws[:, cols].T), bits
    # zero input → exact zeros; linearity
    z = Q.rwkvq_sb6_gemv(dev(np.zeros((1, IN), np.float32)), dev(qblk), dev(qsqm), dev(ddm), OUT, IN, xb)
    assert z.abs().max().item() == 0.0


@pytest.mark.parametrize("bits", [8, 6])
@pytest.mark.parametrize("OUT,IN", [(768, 768), (3072, 768), (768, 3072), (16, 256), (32, 7168)])
def test_sym_gemv_matches_fp64(orc, bits, OUT, IN):
    case(f"sym gemv {OUT}x{IN} bits={bits}")
    qblk, qs, d = sym_tensor(orc, OUT, IN, bits, seed=OUT + bits)
    rng = np.random.default_rng(7)
    for N in (1, 2, 4, 5):
        x = rng.standard_normal((N, IN)).astype(np.float32)
        y = Q.rwkvq_sym_gemv(dev(x), dev(qblk), dev(qs), dev(d), OUT, IN, bits)
        want = orc.sym_gemv_f64(x, qblk, qs, d.view(np.uint16), OUT, IN, bits)
        assert rel(want, y.cpu().numpy()) < GEMV_TOL, N


@pytest.mark.parametrize("xbits", [0, 1, 2])
def test_fused_sb6_gemv_equals_separate_bitwise(orc, xbits):
    case(f"fused sb6 r/k/v xbits={xbits}")
    OUT, IN, Kn = 768, 768, 3
    parts = [sb6_tensor(orc, OUT, IN, xbits, seed=xbits * 10 + i) for i in range(Kn)]
    qblk, qsqm, ddm = (np.concatenate([p[j] for p in parts]) for j in range(3))
    rng = np.random.default_rng(22)
    for N in (1, 2):
        x = rng.standard_normal((N * Kn, IN)).astype(np.float32)
        _lib.reset_counters()
        fused = Q.rwkvq_sb6_gemv(dev(x), dev(qblk), dev(qsqm), dev(ddm), OUT * Kn, IN, xbits, out_per=OUT)
        assert _lib.counters()["sb6_fused"] == 1
        assert fused.shape == (N, OUT * Kn)
        for i, p in enumerate(parts):
            xi = x.reshape(N, Kn, IN)[:, i]
            alone = Q.rwkvq_sb6_gemv(dev(xi), *[dev(z) for z in p], OUT, IN, xbits)
            assert torch.equal(fused[:, i * OUT:(i + 1) * OUT], alone)
    with pytest.raises(ValueError):
        Q.rwkvq_sb6_gemv(dev(x[:2]), dev(qblk), dev(qsqm), dev(ddm), OUT * Kn, IN, xbits, out_per=OUT)


@pytest.mark.parametrize("bits", [8, 6])
def test_fused_sym_gemv_equals_separate_bitwise(orc, bits):
    case(f"fused r/k/v bits={bits}")
    OUT, IN, Kn = 768, 768, 3
    parts = [sym_tensor(orc, OUT, IN, bits, seed=bits * 10 + i) for i in range(Kn)]
    qblk = np.concatenate([p[0] for p in parts])
    qs = np.concatenate([p[1] for p in parts])
    d = np.concatenate([p[2] for p in parts])
    x = np.random.default_rng(21).standard_normal((Kn, IN)).astype(np.float32)
    fused = Q.rwkvq_sym_gemv(dev(x), dev(qblk), dev(qs), dev(d), OUT * Kn, IN, bits, out_per=OUT)
    assert fused.shape == (1, OUT * Kn)
    for i, p in enumerate(parts):
        alone = Q.rwkvq_sym_gemv(dev(x[i:i + 1]), *[dev(z) for z in p], OUT, IN, bits)
        assert torch.equal(fused[:, i * OUT:(i + 1) * OUT], alone)
    want = orc.sym_gemv_f64(x, qblk, qs, d.view(np.uint16), OUT * Kn, IN, bits, out_per=OUT)
    assert rel(want, fused.cpu().numpy()) < GEMV_TOL


# batches run in their own kernel (one weight pass for 2, 4 or 8 inputs, the
# inputs staged in LDS chunk by chunk); 256 x 14336 stages 7 passes of 64
# units in chunks (a partial last chunk); 3072 x 4096 takes tiles of 8 inputs
# at N = 17 / 33 (a grid of >= 1024 workgroups) and of 4 at N = 16; N = 2 and
# N = 5 take tiles of 2
BATCH_NS = (2, 5, 16, 17, 33)


@pytest.mark.parametrize("fmt", ["sb6:0", "sb6:1", "sb6:2", "sym:8", "sym:6"])
@pytest.mark.parametrize("OUT,IN", [(768, 768), (256, 14336), (3072, 4096)])
def test_batched_gemv_rows_equal_single_bitwise(orc, fmt, OUT, IN):
    kind, b = fmt.split(":")
    b = int(b)
    case(f"batched gemv {fmt} {OUT}x{IN}")
    rng = np.random.default_rng(OUT + b)
    if kind == "sb6":
        w = [dev(z) for z in sb6_tensor(orc, OUT, IN, b, seed=OUT + IN + b)]
        run = lambda x: Q.rwkvq_sb6_gemv(x, *w, OUT, IN, b)
        f64 = lambda x: orc.sb6_gemv_f64(x, *[z.cpu().numpy() for z in w[:2]], w[2].cpu().numpy().view(np.uint16),
                                         OUT, IN, b)
    else:
        w = [dev(z) for z in sym_tensor(orc, OUT, IN, b, seed=OUT + b)]
        run = lambda x: Q.rwkvq_sym_gemv(x, *w, OUT, IN, b)
        f64 = lambda x: orc.sym_gemv_f64(x, *[z.cpu().numpy() for z in w[:2]], w[2].cpu().numpy().view(np.uint16),
                                         OUT, IN, b)
    x = rng.standard_normal((max(BATCH_NS), IN)).astype(np.float32)
    single = torch.cat([run(dev(x[n:n + 1])) for n in range(max(BATCH_NS))])
    assert rel(f64(x), single.cpu().numpy()) < GEMV_TOL
    for N in BATCH_NS:
        y = run(dev(x[:N]))
        assert y.shape == (N, OUT)
        assert torch.equal(y, single[:N]), N


def test_batched_fused_gemv_equals_separate_bitwise(orc):
    case("batched fused sb6 r/k/v 3x512x2048")
    OUT, IN, Kn, N = 512, 2048, 3, 16
    parts = [sb6_tensor(orc, OUT, IN, 0, seed=40 + i) for i in range(Kn)]
    qblk, qsqm, ddm = (np.concatenate([p[j] for p in parts]) for j in range(3))
    x = np.random.default_rng(23).standard_normal((N * Kn, IN)).astype(np.float32)
    fused = Q.rwkvq_sb6_gemv(dev(x), dev(qblk), dev(qsqm), dev(ddm), OUT * Kn, IN, 0, out_per=OUT)
    assert fused.shape == (N, OUT * Kn)
    for i, p in enumerate(parts):
        xi = np.ascontiguousarray(x.reshape(N, Kn, IN)[:, i])
        alone = Q.rwkvq_sb6_gemv(dev(xi[:1]), *[dev(z) for z in p], OUT, IN, 0)
        assert torch.equal(fused[:1, i * OUT:(i + 1) * OUT], alone)
        batch = Q.rwkvq_sb6_gemv(dev(xi), *[dev(z) for z in p], OUT, IN, 0)
        assert torch.equal(fused[:, i * OUT:(i + 1) * OUT], batch)


def test_gemv_is_deterministic(orc):
    case("gemv determinism")
    qblk, qsqm, ddm = sb6_tensor(orc, 3072, 768, 1, seed=3)
    x = dev(np.random.default_rng(0).standard_normal((2, 768)).astype(np.float32))
    a = Q.rwkvq_sb6_gemv(x, dev(qblk), dev(qsqm), dev(ddm), 3072, 768, 1)
    b = Q.rwkvq_sb6_gemv(x, dev(qblk), dev(qsqm), dev(ddm), 3072, 768, 1)
    assert torch.equal(a, b)
    # a row of a batch equals the same row alone
    c = Q.rwkvq_sb6_gemv(x[1:2], dev(qblk), dev(qsqm), dev(ddm), 3072, 768, 1)
    assert torch.equal(a[1:2], c)


# ───────────────────────────── sidecar end to end ─────────────────────────────

def synth_file(path, kind, bits):
    rng = np.random.default_rng(42)
    tensors = {}
    for l in range(2):
        for m in ("receptance", "key", "value", "output"):
            w = (rng.standard_normal((256, 256)) * 0.02).astype(np.float32)
            tensors[f"blocks.{l}.att.{m}.weight"] = Q.sb6_entry(w, bits) if kind == "sb6" else Q.sym_entry(w, bits)
        w = (rng.standard_normal((1024, 256)) * 0.02).astype(np.float32)
        tensors[f"blocks.{l}.ffn.key.weight"] = Q.sb6_entry(w, bits) if kind == "sb6" else Q.sym_entry(w, bits)
    ln = (rng.standard_normal(256)).astype(np.float32)
    tensors["ln_out.weight"] = ({"kind": "dense", "shape": [256]}, {"dense": ln})
    Q.write_rwkvq(path, tensors, n_layer=2, n_embd=256, vocab_size=1024)
    return tensors


@pytest.mark.parametrize("kind,bits", [("sb6", 4), ("sb6", 6), ("sym", 8), ("sym", 6)])
def test_sidecar_end_to_end(tmp_path, orc, kind, bits):
    case(f"sidecar {kind}{bits}")
    p = str(tmp_path / f"{kind}{bits}.rwkvq")
    synth_file(p, kind, bits)
    groups = {"att0": [f"blocks.0.att.{m}.weight" for m in ("receptance", "key", "value")]}
    sc = Q.RwkvqSidecar.from_rwkvq(p, fusing_sym=groups)
    key = "blocks.1.att.key.weight"
    info = sc.tensors[key]
    deq = sc.dequantize(key)
    if kind == "sb6":
        want = orc.sb6_dequant(*[sc.arrays[f"{key}::{f}"].cpu().numpy() for f in ("qblk", "qsqm")],
                               sc.arrays[f"{key}::ddm"].view(torch.int16).cpu().numpy().view(np.uint16),
                               256, 256, info.xbits)
    else:
        want = orc.sym_dequant(sc.arrays[f"{key}::qblk"].cpu().numpy(), sc.arrays[f"{key}::qs"].cpu().numpy(),
                               sc.arrays[f"{key}::d"].view(torch.int16).cpu().numpy().view(np.uint16), 256, 256, bits)
    assert np.array_equal(deq.cpu().numpy(), want)
    assert torch.equal(sc.dequantize(key, torch.bfloat16), deq.to(torch.bfloat16))
    x = torch.randn((1, 256), device=DEV, generator=torch.Generator(DEV).manual_seed(0))
    y = sc.sb6_gemv(key, x) if kind == "sb6" else sc.sym_gemv(key, x)
    assert y is not None
    assert rel((x.double() @ deq.double().T).cpu().numpy(), y.cpu().numpy()) < GEMV_TOL
    # declines what it cannot take (RwkvqSb6GEMVTests.swift:88-100)
    other = sc.sym_gemv if kind == "sb6" else sc.sb6_gemv
    assert other(key, x) is None
    assert (sc.sb6_gemv if kind == "sb6" else sc.sym_gemv)(key, torch.zeros((1, 128), device=DEV)) is None
    if kind == "sb6":
        assert sc.sb6_gemv(key, torch.zeros((2, 256), device=DEV)) is None
        assert not sc.sym_fused
        sf = sc.fusing_sb6(groups)
        assert set(sf.sb6_fused) == {"att0"}
        xs = torch.randn((3, 256), device=DEV)
        fused = sf.sb6_gemv_fused("att0", xs)
        for i, k in enumerate(groups["att0"]):
            assert torch.equal(fused[i:i + 1], sf.sb6_gemv(k, xs[i:i + 1]))
            assert torch.equal(sf.dequantize(k), sc.dequantize(k))
        assert sf.sb6_gemv_fused("att0", torch.zeros((2, 256), device=DEV)) is None
        assert not sf.fusing_sb6({"x": ["blocks.0.att.key.weight", "blocks.0.ffn.key.weight"]}).sb6_fused.keys() - {"att0"}
    else:
        assert sc.sym_gemv(key, torch.zeros((5, 256), device=DEV)) is None
        assert set(sc.sym_fused) == {"att0"}
        xs = torch.randn((3, 256), device=DEV)
        fused = sc.sym_gemv_fused("att0", xs)
        for i, k in enumerate(groups["att0"]):
            assert torch.equal(fused[i:i + 1], sc.sym_gemv(k, xs[i:i + 1]))
        assert sc.sym_gemv_fused("att0", torch.zeros((2, 256), device=DEV)) is None
        assert sc.sym_gemv_fused("none", xs) is None
    assert torch.equal(sc.dequantize("ln_out.weight"), sc.arrays["ln_out.weight::dense"].float())


@pytest.mark.parametrize("kind,bits", [("sb6", 4), ("sb6", 6), ("sym", 8), ("sym", 6)])
def test_base_proj_paths(tmp_path, orc, kind, bits):
    """The .rwkvq branch of baseProj: GEMV on decode / short passes, dequantise
    + matmul in the base dtype otherwise, the result in the input's dtype."""
    case(f"base_proj {kind}{bits}")
    p = str(tmp_path / f"{kind}{bits}.rwkvq")
    synth_file(p, kind, bits)
    sc = Q.RwkvqSidecar.from_rwkvq(p)
    key = "blocks.1.ffn.key.weight"   # 1024 x 256
    W = sc.dequantize(key).double()
    gen = torch.Generator(DEV).manual_seed(3)
    x = torch.randn((2, 5, 256), device=DEV, generator=gen)
    want = (x.double() @ W.T).cpu().numpy()
    gemv = Q.rwkvq_sb6_gemv if kind == "sb6" else Q.rwkvq_sym_gemv
    fields = ("qblk", "qsqm", "ddm") if kind == "sb6" else ("qblk", "qs", "d")
    code = sc.tensors[key].xbits if kind == "sb6" else bits
    direct = gemv(x.reshape(10, 256), *[sc.arrays[f"{key}::{f}"] for f in fields], 1024, 256, code)
    # decode and short passes: the kernel, all ten rows in one launch
    for kw in ({"decode": True}, {"short_rows": 10}):
        y = sc.base_proj(key, x, **kw)
        assert y.shape == (2, 5, 1024) and y.dtype == torch.float32
        assert torch.equal(y.reshape(10, 1024), direct), kw
        assert rel(want, y.cpu().numpy()) < GEMV_TOL
    # longer than the short-pass threshold: the fp16 long pass on the matrix
    # cores (the fp16 dequant's weights, fp16 inputs, the fp16 rounding of an
    # fp32 sum); bf16: dequantise + matmul in bf16
    from tests.test_gpu_prefill import check_f16_rounding
    y = sc.base_proj(key, x, base_dtype=torch.float16, short_rows=9)
    assert y.dtype == torch.float32
    w16 = sc.dequantize(key, torch.float16).double().cpu().numpy()
    x16 = x.reshape(10, 256).to(torch.float16).double().cpu().numpy()
    check_f16_rounding(y.reshape(10, 1024).cpu().numpy(), x16 @ w16.T, np.abs(x16) @ np.abs(w16).T)
    assert rel(want, y.cpu().numpy()) < 2e-3
    y = sc.base_proj(key, x, base_dtype=torch.bfloat16, short_rows=9)
    ref = torch.nn.functional.linear(x.reshape(10, 256).to(torch.bfloat16), sc.dequantize(key, torch.bfloat16)).float()
    assert torch.equal(y.reshape(10, 1024), ref)
    assert rel(want, y.cpu().numpy()) < 1e-2
    # the output takes the input's dtype
    xb = x.to(torch.bfloat16)
    assert sc.base_proj(key, xb, decode=True).dtype == torch.bfloat16
    assert sc.base_proj(key, xb).dtype == torch.bfloat16
    assert Q.default_short_pass_rows(768, sym=False) == 4
    assert Q.default_short_pass_rows(2048, sym=True) == 16
    with pytest.raises(ValueError):
        sc.base_proj(key, torch.zeros((1, 128), device=DEV))


@pytest.mark.parametrize("bits", [8, 6])
def test_sym_rows_equal_dense_rows_bitwise(orc, bits):
    """RwkvqSymRows: the gathered rows are the dense table's rows, bitwise."""
    case(f"sym rows bits={bits}")
    OUT, IN = 1000, 256 + 128 * (bits == 8)   # IN off the 256 super-block for 8 bits
    qblk, qs, d = (dev(z) for z in sym_tensor(orc, OUT, IN, bits, seed=50 + bits))
    ids = torch.tensor([[0, 999, 17], [17, 500, 3]], device=DEV)
    for dt in (torch.float16, torch.bfloat16, torch.float32):
        dense = Q.rwkvq_dequant_sym(qblk, qs, d, OUT, IN, bits, dt)
        _lib.reset_counters()
        rows = Q.rwkvq_sym_rows(ids, qblk, qs, d, OUT, IN, bits, dt)
        assert _lib.counters()["sym_rows"] == 1
        assert rows.shape == (2, 3, IN) and rows.dtype == dt
        assert torch.equal(rows, dense[ids]), dt
    # out-of-range ids give NaN rows; the others are unaffected
    bad = Q.rwkvq_sym_rows(torch.tensor([5, -1, OUT], device=DEV), qblk, qs, d, OUT, IN, bits)
    assert torch.equal(bad[0], Q.rwkvq_dequant_sym(qblk, qs, d, OUT, IN, bits, torch.float16)[5])
    assert torch.isnan(bad[1:]).all()
    assert Q.rwkvq_sym_rows(torch.zeros((0,), dtype=torch.int64, device=DEV), qblk, qs, d, OUT, IN, bits).shape == (0, IN)


def test_sym_row_table_from_sidecar(tmp_path):
    case("sym row table from a .rwkvq file")
    p8, p6 = str(tmp_path / "s8.rwkvq"), str(tmp_path / "s6.rwkvq")
    synth_file(p8, "sym", 8)
    synth_file(p6, "sym", 6)
    sc8, sc6 = Q.RwkvqSidecar.from_rwkvq(p8), Q.RwkvqSidecar.from_rwkvq(p6)
    key = "blocks.0.ffn.key.weight"
    t = sc8.sym_row_table(key)
    assert t is not None and t.row_count == 1024 and t.in_features == 256
    ids = torch.tensor([3, 1023, 3, 0], device=DEV)
    assert torch.equal(t.rows(ids), t.dense()[ids])
    assert torch.equal(t.dense(), sc8.dequantize(key, torch.float16))
    assert t.packed_bytes == 1024 * 256 + 1024 * 16 + 1024 * 2
    # the reference declines 6-bit tables and non-sym tensors (RwkvqSymRows.swift:70-80)
    assert sc6.sym_row_table(key) is None
    assert sc8.sym_row_table("ln_out.weight") is None
    assert sc8.sym_row_table("missing") is None
