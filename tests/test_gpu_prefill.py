"""GPU parity of the parallel-pass (prefill) path.

The sb6 matrix-core GEMM against the fp16-base long pass of the reference
(X070Backbone.baseMatmul, X070Backbone.swift:337-356): every output is the
fp16 rounding of an fp32-accurate sum of the exact products of the fp16
inputs and fp16 dequantised weights: within ½ fp16 ulp plus 2^-16·Σ|x·w| of
the exact value, and equal to its fp16 rounding for all but a small fraction
of outputs.  Epilogues and
fused groups are bitwise the plain launch and the separate operations; rows
are independent of the other rows of the launch (bitwise).
"""
import sys

import numpy as np
import pytest
import torch

from swiftrwkv_amd import quant as Q
from tests.test_gpu_model_shapes import random_k3

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def check_f16_rounding(got, exact, mag):
    """got = fp16(acc) with |acc − exact| ≤ 2^-16·Σ|x·w| (an fp32 sum of the
    same products): |got − exact| ≤ ½ ulp16 + 2^-16·mag everywhere.  Returns
    the fraction of outputs that differ from fp16(exact)."""
    got = np.asarray(got, np.float64)
    assert np.all(np.isfinite(got))
    ulp = np.maximum(np.spacing(np.abs(got).astype(np.float16)).astype(np.float64),
                     np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64))
    excess = np.abs(got - exact) - (0.5 * ulp + 2.0 ** -16 * mag)
    assert excess.max() <= 0, f"worst excess {excess.max():.3e} at {np.unravel_index(excess.argmax(), excess.shape)}"
    return float((got != exact.astype(np.float16).astype(np.float64)).mean())


@pytest.mark.parametrize("M,OUT,IN", [(1, 256, 256), (37, 768, 768), (300, 3072, 768), (128, 768, 3072),
                                      (257, 4096, 1024), (130, 1024, 4096)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.float16])
def test_sb6_gemm_matches_f16_base_pass(orc, M, OUT, IN, xdt):
    case(f"sb6 gemm M={M} {OUT}x{IN} x {xdt}")
    rng = np.random.default_rng(M + OUT + IN)
    qblk, qsqm, ddm = random_k3(OUT, IN, rng)
    x = rng.standard_normal((M, IN)).astype(np.float32)
    if xdt == torch.float16:
        x = x.astype(np.float16).astype(np.float32)
    y = Q.rwkvq_sb6_gemm(dev(x).to(xdt), dev(qblk), dev(qsqm), dev(ddm), OUT, IN)
    exact, mag = orc.sb6_matmul_f16_base(x, qblk, qsqm, ddm.view(np.uint16), OUT, IN)
    frac = check_f16_rounding(y.cpu().numpy(), exact, mag)
    print(f"[gemm] M={M} {OUT}x{IN}: {frac:.2e} of outputs on the other side of an fp16 boundary", flush=True)
    assert frac < 5e-2


def quant_matrix(orc, fmt, OUT, IN, rng):
    """A random matrix of layout `fmt` ("sb6:<xbits>", "sym:<bits>") in the
    loader layout, with the oracle's fp16-base product of it."""
    from tests.test_gpu_rwkvq import sb6_tensor, sym_tensor
    kind, b = fmt.split(":")
    b = int(b)
    seed = int(rng.integers(0, 1 << 30))
    if kind == "sb6":
        bufs = sb6_tensor(orc, OUT, IN, b, seed)
        base = lambda x: orc.sb6_matmul_f16_base(x, bufs[0], bufs[1], bufs[2].view(np.uint16), OUT, IN, b)
        gemm = lambda x, w, **kw: Q.rwkvq_sb6_gemm(x, *w, OUT, IN, b, **kw)
    else:
        bufs = sym_tensor(orc, OUT, IN, b, seed)
        base = lambda x: orc.sym_matmul_f16_base(x, bufs[0], bufs[1], bufs[2].view(np.uint16), OUT, IN, b)
        gemm = lambda x, w, **kw: Q.rwkvq_sym_gemm(x, *w, OUT, IN, b, **kw)
    return bufs, base, gemm


@pytest.mark.parametrize("fmt", ["sb6:1", "sb6:2", "sym:8", "sym:6"])
@pytest.mark.parametrize("M,OUT,IN", [(1, 256, 256), (37, 768, 768), (300, 3072, 768), (130, 1024, 4096)])
def test_quant_gemm_layouts_match_f16_base_pass(orc, fmt, M, OUT, IN):
    """The long pass of the other layouts (sb6 5 / 6-bit, sym 8 / 6-bit) on
    the matrix cores against the fp16-base oracle (the fp16 dequant's
    weights, fp16 inputs, an exact sum): within ½ fp16 ulp + 2^-16·Σ|x·w|;
    fp16 inputs equal fp32 inputs holding the same values."""
    case(f"quant gemm {fmt} M={M} {OUT}x{IN}")
    rng = np.random.default_rng(M * 7 + OUT + IN)
    bufs, base, gemm = quant_matrix(orc, fmt, OUT, IN, rng)
    w = [dev(z) for z in bufs]
    x = rng.standard_normal((M, IN)).astype(np.float32)
    y = gemm(dev(x), w)
    exact, mag = base(x)
    frac = check_f16_rounding(y.cpu().numpy(), exact, mag)
    print(f"[gemm] {fmt} M={M} {OUT}x{IN}: {frac:.2e} of outputs on the other side of an fp16 boundary", flush=True)
    assert frac < 5e-2
    x16 = dev(x).to(torch.float16)
    assert torch.equal(gemm(x16, w), gemm(x16.float(), w))


@pytest.mark.parametrize("fmt", ["sb6:2", "sym:6"])
@pytest.mark.parametrize("split", [False, True])
def test_quant_gemm_layouts_epilogues_and_groups(orc, fmt, split):
    """One K range: fused groups equal their members bitwise and rows do not
    depend on the other rows of the launch.  Split K sums (a few tiles): the
    fp16-base oracle's bound (the sum's order is not the one range's),
    deterministic.  Either way the add / relu² epilogues are the separate
    operations' arithmetic."""
    case(f"quant gemm {fmt} epilogues, groups, rows, split {split}")
    D, M = 512, 150
    rng = np.random.default_rng(17)
    bufs, base_pass, _ = quant_matrix(orc, fmt, 3 * D, D, rng)
    w = [dev(z) for z in bufs]
    kind, b = fmt.split(":")
    entry = Q.rwkvq_sb6_gemm if kind == "sb6" else Q.rwkvq_sym_gemm
    assert Q.rwkvq_gemm_workspace(M, 3 * D, D) > 0 and Q.rwkvq_gemm_workspace(M, D, D) > 0
    x = dev(rng.standard_normal((3, M, D)).astype(np.float32))
    fused = entry(x, *w, 3 * D, D, int(b), out_per=D, split=split)
    for g in range(3):
        rows = slice(g * D, (g + 1) * D)
        part = [z[rows] for z in w]
        sep = entry(x[g], *part, D, D, int(b), split=split)
        one = entry(x[g], *part, D, D, int(b), split=False)
        if split:
            exact, mag = base_pass(x[g].cpu().numpy())
            for got in (fused[:, rows], sep):
                frac = check_f16_rounding(got.cpu().numpy(), exact[:, rows], mag[:, rows])
                assert frac < 5e-2
            assert torch.equal(entry(x[g], *part, D, D, int(b), split=True), sep)
            assert not torch.equal(sep, one)   # the split ran (a different sum order somewhere)
            continue
        assert torch.equal(fused[:, rows], sep), g
        for m in (0, 77, 149):
            assert torch.equal(entry(x[g, m:m + 1], *part, D, D, int(b), split=False)[0], sep[m])
    part = [z[:D] for z in w]
    y0 = entry(x[1], *part, D, D, int(b), split=split)
    base = dev(rng.standard_normal((M, D)).astype(np.float32))
    y1 = base.clone()
    entry(x[1], *part, D, D, int(b), epilogue="add", out=y1, split=split)
    assert torch.equal(y1, base + y0)
    h = entry(x[1], *part, D, D, int(b), epilogue="relu2_f16", split=split)
    assert h.dtype == torch.float16 and torch.equal(h, (torch.relu(y0) * torch.relu(y0)).to(torch.float16))


def test_quant_gemm_split_workspace_contract(orc):
    """The split long pass through the C-ABI: a workspace smaller than
    rwkv_quant_gemm_workspace is refused (nothing launched, y untouched), a
    NULL one runs as one K range, an adequate one gives the split sums."""
    case("quant gemm workspace contract")
    from swiftrwkv_amd import _lib
    M, OUT, IN = 96, 768, 3072
    rng = np.random.default_rng(19)
    bufs, base, gemm = quant_matrix(orc, "sb6:0", OUT, IN, rng)
    w = [dev(z) for z in bufs]
    x = dev(rng.standard_normal((M, IN)).astype(np.float32))
    need = Q.rwkvq_gemm_workspace(M, OUT, IN)
    assert need >= 2 * M * OUT * 4
    L, s = _lib.lib(), torch.cuda.current_stream().cuda_stream
    y = torch.full((M, OUT), 3.0, device=DEV)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    args = lambda: (x.data_ptr(), _lib.F32, M, IN, M * IN, *[b.data_ptr() for b in w], y.data_ptr(), OUT, OUT, IN, 0,
                    OUT, 0)
    assert L.rwkv_sb6_gemm(*args(), ws.data_ptr(), need - 16, s) != 0
    torch.cuda.synchronize()
    assert torch.all(y == 3.0)
    _lib.check(L.rwkv_sb6_gemm(*args(), None, 0, s))
    assert torch.equal(y, gemm(x, w, split=False))
    _lib.check(L.rwkv_sb6_gemm(*args(), ws.data_ptr(), need, s))
    assert torch.equal(y, gemm(x, w, split=True))
    exact, mag = base(x.cpu().numpy())
    check_f16_rounding(y.cpu().numpy(), exact, mag)


@pytest.mark.parametrize("fmt", ["sb6:0", "sb6:2", "sym:8", "sym:6"])
def test_quant_gemm_dense_route_bitwise(orc, fmt):
    """Shapes with at least 128 output tiles of 256 × 256 and fp16 inputs:
    given a workspace, the quantised entry points dequantise the weight into
    it and run the dense fp16 kernel — bitwise the one-range fused launch
    (the same products in the same order) for a fused group of three
    matrices with a partial last row block, for every epilogue; and within
    the fp16-base oracle's bound on a sample of rows."""
    case(f"quant gemm dense route {fmt}")
    from swiftrwkv_amd import _lib
    M, D, IN = 2000, 1536, 512   # 8 row blocks × 18 feature blocks
    rng = np.random.default_rng(23)
    bufs, base_pass, _ = quant_matrix(orc, fmt, 3 * D, IN, rng)
    w = [dev(z) for z in bufs]
    kind, b = fmt.split(":")
    entry = Q.rwkvq_sb6_gemm if kind == "sb6" else Q.rwkvq_sym_gemm
    dq = "sb6_dequant" if kind == "sb6" else "sym_dequant"
    assert Q.rwkvq_gemm_workspace(M, 3 * D, IN) == 3 * D * IN * 2
    x = dev(rng.standard_normal((3, M, IN)).astype(np.float32)).to(torch.float16)
    n0 = _lib.counters()[dq]
    dense = entry(x, *w, 3 * D, IN, int(b), out_per=D, split=True)
    assert _lib.counters()[dq] == n0 + 1   # the dense route ran
    one = entry(x, *w, 3 * D, IN, int(b), out_per=D, split=False)
    assert _lib.counters()[dq] == n0 + 1
    assert torch.equal(dense, one)
    base = dev(rng.standard_normal((M, 3 * D)).astype(np.float32))
    y1 = base.clone()
    entry(x, *w, 3 * D, IN, int(b), out_per=D, epilogue="add", out=y1, split=True)
    assert torch.equal(y1, base + one)
    h = entry(x, *w, 3 * D, IN, int(b), out_per=D, epilogue="relu2_f16", split=True)
    assert torch.equal(h, (torch.relu(one) * torch.relu(one)).to(torch.float16))
    rows = np.r_[0:24, M - 24:M]
    for g in range(3):
        exact, mag = base_pass(x[g].float().cpu().numpy()[rows])
        cols = slice(g * D, (g + 1) * D)
        assert check_f16_rounding(dense[rows][:, cols].cpu().numpy(), exact[:, cols], mag[:, cols]) < 5e-2


@pytest.mark.parametrize("M", [1, 257, 1000])
def test_f16_gemm_matches_exact_products(M):
    """rwkv_f16_gemm on a dense fp16 weight: every output within ½ fp16 ulp +
    2^-16·Σ|x·w| of the exact product of the fp16 operands; a fused pair of
    matrices equals its members; shapes off the 256-feature tiles refused."""
    case(f"f16 gemm M={M}")
    rng = np.random.default_rng(M)
    OUT, IN = 768, 384
    x = (rng.standard_normal((M, IN)) * 0.5).astype(np.float16)
    wt = (rng.standard_normal((OUT, IN)) * 0.1).astype(np.float16)
    y = Q.rwkvq_f16_gemm(dev(x), dev(wt))
    xd, wd = x.astype(np.float64), wt.astype(np.float64)
    check_f16_rounding(y.cpu().numpy(), xd @ wd.T, np.abs(xd) @ np.abs(wd).T)
    w2 = np.concatenate([wt, wt[::-1].copy()])
    x2 = np.stack([x, x[::-1].copy()])
    pair = Q.rwkvq_f16_gemm(dev(x2), dev(w2), out_per=OUT)
    assert torch.equal(pair[:, :OUT], y)
    assert torch.equal(pair[:, OUT:], Q.rwkvq_f16_gemm(dev(x2[1]), dev(wt[::-1].copy())))
    assert not Q.rwkvq_f16_gemm_applies(M, 640, IN) and not Q.rwkvq_f16_gemm_applies(M, OUT, 320)
    with pytest.raises(ValueError):
        Q.rwkvq_f16_gemm(dev(x[:, :320].copy()), dev(wt[:, :320].copy()))


@pytest.mark.parametrize("D,M,ranks,wdt", [(256, 37, (32, 32, 32, 64), torch.float16),
                                             (768, 512, (16, 32, 16, 64), torch.float16),
                                             (768, 513, (16, 32, 16, 64), torch.float32),
                                             (1024, 200, (64, 64, 32, 128), torch.float32),
                                             (4096, 70, (128, 128, 96, 480), torch.float16),
                                             (1024, 2100, (64, 64, 32, 160), torch.float16),
                                             (4096, 600, (128, 128, 96, 480), torch.float16),
                                             (2048, 1100, (96, 96, 64, 256), torch.float32)])
@pytest.mark.parametrize("with_v", [1, 0])
def test_seq_lora_matches_fp64(D, M, ranks, wdt, with_v):
    """The parallel pass's four low-rank branches (rwkv_x070_seq_lora) against
    fp64 products of the same values: ww = tanh(x_w·A_wᵀ)·B_wᵀ, aa, vv (not
    written when the layer has no v branch), gate = sigmoid(x_g·A_gᵀ)·B_gᵀ.
    Long passes with fp16 matrices (M·D above 2^21) take the two-part fp16
    kernel: the same bound (its activations keep 22 of 24 bits); odd stage
    counts (ranks 96, 160) and partial row / column tiles included.  Up to
    512 rows the K-split kernel runs (ranks 16 and 32 leave some of its
    waves without K steps); 513 rows take the 64 × 64 tiles."""
    case(f"seq lora D={D} M={M} ranks={ranks} {wdt} with_v={with_v}")
    from swiftrwkv_amd import _lib
    rng = np.random.default_rng(D + M + with_v)
    rw, ra, rv, rg = ranks
    wcode = _lib.F16 if wdt == torch.float16 else _lib.F32
    assert bool(_lib.lib().rwkv_x070_seq_lora_split(M, D, wcode, *ranks)) == (wdt == torch.float16 and M * D > 1 << 21)
    RT = sum(ranks)
    mix = rng.standard_normal((6, M, D)).astype(np.float32)
    A = (rng.standard_normal((RT, D)) / np.sqrt(D)).astype(np.float32)
    Bs = [(rng.standard_normal((D, r)) * 0.5 / np.sqrt(r)).astype(np.float32) for r in ranks]
    A_d = dev(A).to(wdt)
    B_d = [dev(b).to(wdt) for b in Bs]
    A64 = A_d.double().cpu().numpy()
    B64 = [b.double().cpu().numpy() for b in B_d]
    la = torch.empty((M, RT), device=DEV)
    outs = [torch.full((M, D), 7.0, device=DEV) for _ in range(4)]
    L = _lib.lib()
    mix_d = dev(mix)   # held: the kernels run after the call returns
    _lib.check(L.rwkv_x070_seq_lora(mix_d.data_ptr(), M, D, A_d.data_ptr(), *[b.data_ptr() for b in B_d],
                                    _lib.F16 if wdt == torch.float16 else _lib.F32, rw, ra, rv, rg, with_v,
                                    la.data_ptr(), *[o.data_ptr() for o in outs], torch.cuda.current_stream().cuda_stream))
    x = mix.astype(np.float64)
    offs = np.cumsum((0,) + ranks)
    inner = [x[c] @ A64[offs[b]:offs[b + 1]].T for b, c in enumerate((3, 4, 2, 5))]
    acts = [np.tanh(inner[0]), inner[1], inner[2], 1.0 / (1.0 + np.exp(-inner[3]))]
    want = [acts[b] @ B64[b].T for b in range(4)]
    for b, name in enumerate(("ww", "aa", "vv", "gate")):
        got = outs[b].cpu().numpy()
        if b == 2 and not with_v:
            assert np.all(got == 7.0), name   # layer 0: no v branch, vv untouched
            continue
        err = rel(want[b], got)
        print(f"[seq lora] D={D} M={M} {name}: rel {err:.2e}", flush=True)
        assert err < 2e-5, name


@pytest.mark.parametrize("nc,f16", [(6, False), (1, True)])
def test_seq_shift_mix_updates_state_in_place(nc, f16):
    """rwkv_x070_seq_shift_mix with prev_out = prev_in (how the parallel pass
    calls it): the carried state of each row becomes xl of its last real
    token (rwkvTokenShift's gatherLast) and stays as it was for a row with no
    tokens, bitwise as with separate buffers; t = 0 lerps against the old
    state, t > 0 against the previous row."""
    case(f"seq shift mix in place nc={nc} f16={f16}")
    from swiftrwkv_amd import _lib
    B, T, D = 4, 9, 256
    rng = np.random.default_rng(nc)
    xl = rng.standard_normal((B * T, D)).astype(np.float32)
    prev = rng.standard_normal((B, D)).astype(np.float32)
    coef = rng.random((nc, D)).astype(np.float32)
    lens = np.array([T, 1, T - 3, 0], dtype=np.int32)
    outs = {}
    xl_d, lens_d, coef_d = dev(xl), dev(lens), dev(coef)   # held: the kernel runs after the call returns
    for alias in (True, False):
        st = dev(prev)
        dst = st if alias else torch.full((B, D), 5.0, device=DEV)
        if not alias:
            dst[3] = st[3]   # a row with no tokens keeps its state
        y0 = torch.empty((B * T, nc, D), dtype=torch.float16 if f16 else torch.float32, device=DEV)
        _lib.check(_lib.lib().rwkv_x070_seq_shift_mix(
            xl_d.data_ptr(), st.data_ptr(), dst.data_ptr(), lens_d.data_ptr(), coef_d.data_ptr(), nc, nc,
            y0.data_ptr(), _lib.F16 if f16 else _lib.F32, nc * D, D, None, 0, 0, 0, B, T, D,
            torch.cuda.current_stream().cuda_stream))
        outs[alias] = (dst.cpu().numpy(), y0.float().cpu().numpy())
    assert np.array_equal(outs[True][0], outs[False][0])
    assert np.array_equal(outs[True][1], outs[False][1])
    want_state = prev.copy()
    for b in range(3):
        want_state[b] = xl[b * T + lens[b] - 1]
    assert np.array_equal(outs[True][0], want_state)
    x = xl.reshape(B, T, D).astype(np.float64)
    p = np.concatenate([prev[:, None].astype(np.float64), x[:, :-1]], axis=1)
    want = x[:, :, None] + (p - x)[:, :, None] * coef.astype(np.float64)[None, None]
    got = outs[True][1].reshape(B, T, nc, D)
    tol = 2e-3 if f16 else 1e-6
    assert np.abs(got - want).max() <= tol * max(1.0, np.abs(want).max())


def test_sb6_gemm_epilogues_groups_and_row_independence(orc):
    case("sb6 gemm epilogues, r/k/v group, rows")
    D, M = 1024, 200
    rng = np.random.default_rng(7)
    qblk, qsqm, ddm = (dev(z) for z in random_k3(3 * D, D, rng))
    x = dev(rng.standard_normal((3, M, D)).astype(np.float32))
    fused = Q.rwkvq_sb6_gemm(x, qblk, qsqm, ddm, 3 * D, D, out_per=D, split=False)
    for g in range(3):
        rows = slice(g * D, (g + 1) * D)
        sep = Q.rwkvq_sb6_gemm(x[g], qblk[rows], qsqm[rows], ddm[rows], D, D, split=False)
        assert torch.equal(fused[:, rows], sep), g
        for m in (0, 63, 199):   # a row alone gives the same bits as inside the launch
            assert torch.equal(Q.rwkvq_sb6_gemm(x[g, m:m + 1], qblk[rows], qsqm[rows], ddm[rows], D, D,
                                                split=False)[0], sep[m])
    base = dev(rng.standard_normal((M, D)).astype(np.float32))
    y0 = Q.rwkvq_sb6_gemm(x[1], qblk[:D], qsqm[:D], ddm[:D], D, D)
    y1 = base.clone()
    Q.rwkvq_sb6_gemm(x[1], qblk[:D], qsqm[:D], ddm[:D], D, D, epilogue="add", out=y1)
    assert torch.equal(y1, base + y0)
    h = Q.rwkvq_sb6_gemm(x[1], qblk[:D], qsqm[:D], ddm[:D], D, D, epilogue="relu2_f16")
    assert h.dtype == torch.float16
    assert torch.equal(h, (torch.relu(y0) * torch.relu(y0)).to(torch.float16))
    # fp16 inputs equal fp32 inputs holding the same fp16 values
    x16 = x[1].to(torch.float16)
    assert torch.equal(Q.rwkvq_sb6_gemm(x16, qblk[:D], qsqm[:D], ddm[:D], D, D),
                       Q.rwkvq_sb6_gemm(x16.float(), qblk[:D], qsqm[:D], ddm[:D], D, D))
    with pytest.raises(ValueError):
        Q.rwkvq_sb6_gemm(x[0], qblk[:D], qsqm[:D], ddm[:D], D + 64, D)


# ───────────────────────── the parallel (prefill) pass of the model ─────────────────────────

from oracle import x070 as X                      # noqa: E402
from swiftrwkv_amd import synthetic as syn        # noqa: E402
from swiftrwkv_amd.x070 import X070Decoder        # noqa: E402

TINY = syn.X070Shape("tiny", 2, 256, 1024, vocab=512)
# lengths around the 16-token chunk of the reference kernels (BatchGenerateTests.swift:29-30)
PROMPTS = [[1, 2, 3, 4, 5], [7, 8, 9, 10, 11, 12, 13, 14, 15], [42], [(i * 5) % 512 for i in range(16)],
           [(i * 3 + 1) % 512 for i in range(17)]]


def rel(ref, got):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(ref - np.asarray(got, np.float64)).max() / (np.abs(ref).max() + 1e-30))


@pytest.fixture(scope="module")
def tiny_model():
    proj = syn.x070_projections(TINY, nthreads=4)
    return proj, X.dequant_projections(proj)


@pytest.mark.parametrize("lora", ["f32", "f16"])
def test_prefill_fp32_base_matches_oracle_and_rows_are_independent(tiny_model, lora):
    """fp32 base (every projection on the fp32 GEMV): each row's last logits
    and states against the oracle's parallel pass of that prompt alone
    (1e-4), and each row against the same prompt prefilled alone (1e-5): the
    pad steps are neutral and rows do not see each other."""
    case(f"prefill fp32 base, low-rank {lora}")
    proj, W = tiny_model
    p = syn.x070_dense_params(TINY, seed=31, lora_dtype=np.float32 if lora == "f32" else np.float16)
    dec = X070Decoder(TINY.n_layer, TINY.n_embd, TINY.ffn, TINY.vocab, p, proj, DEV)
    logits, st = dec.prefill_batch(PROMPTS, base_dtype=torch.float32)
    assert logits.shape == (len(PROMPTS), TINY.vocab)
    for i, pr in enumerate(PROMPTS):
        ref, ost = X.prefill(p, W, pr, TINY.n_layer, TINY.n_head)
        e = rel(ref, logits[i].cpu().numpy())
        ew = rel(ost.wkv[:, 0], st.wkv[:, i].cpu().numpy())
        es = max(rel(ost.tmix_prev[:, 0], st.tmix_prev[:, i].cpu().numpy()),
                 rel(ost.cmix_prev[:, 0], st.cmix_prev[:, i].cpu().numpy()))
        print(f"[prefill] fp32 base row {i} (T={len(pr)}): logits {e:.2e}, wkv {ew:.2e}, shift {es:.2e}", flush=True)
        assert e < 1e-4 and ew < 1e-4 and es < 1e-4, i
        alone, _ = dec.prefill_batch([pr], base_dtype=torch.float32)
        assert rel(alone[0].cpu().numpy(), logits[i].cpu().numpy()) < 1e-5, i


def test_prefill_fp16_base_long_pass_matches_oracle(tiny_model):
    """fp16 base, every projection on the matrix-core long pass: the oracle
    with the same fp16 rounding points (inputs, dequantised weights, product
    outputs, relu²), within the flips an fp32 sum may take at those points."""
    case("prefill fp16 base (matrix-core long pass)")
    proj, W = tiny_model
    p = syn.x070_dense_params(TINY, seed=32, lora_dtype=np.float16)
    dec = X070Decoder(TINY.n_layer, TINY.n_embd, TINY.ffn, TINY.vocab, p, proj, DEV)
    from swiftrwkv_amd import _lib
    n0 = _lib.counters()["sb6_gemm"]
    logits, st = dec.prefill_batch(PROMPTS, base_dtype=torch.float16, short_rows=0)
    assert _lib.counters()["sb6_gemm"] - n0 == TINY.n_layer * 4   # r/k/v, o, ffn key, ffn value
    for i, pr in enumerate(PROMPTS):
        ref, ost = X.prefill(p, W, pr, TINY.n_layer, TINY.n_head, f16_base=True)
        e = rel(ref, logits[i].cpu().numpy())
        ew = rel(ost.wkv[:, 0], st.wkv[:, i].cpu().numpy())
        print(f"[prefill] fp16 base row {i} (T={len(pr)}): logits {e:.2e}, wkv {ew:.2e}", flush=True)
        assert e < 2e-3 and ew < 2e-3, i


def test_prefill_time_chunked_wkv_matches_oracle(tiny_model):
    """The prefill with its WKV-7 pass in 32-token chunks (forced for the
    short prompts, chosen by itself for a 600-token one): the oracle at the
    fp32 bar (1e-4), and the step-by-step pass within fp32 rounding (1e-5)."""
    case("prefill fp32 base, time-chunked WKV")
    from swiftrwkv_amd import _lib
    from swiftrwkv_amd.x070 import wkv_chunked_prefers
    proj, W = tiny_model
    p = syn.x070_dense_params(TINY, seed=35, lora_dtype=np.float32)
    dec = X070Decoder(TINY.n_layer, TINY.n_embd, TINY.ffn, TINY.vocab, p, proj, DEV)
    n0 = _lib.counters()["seq_chunked"]
    logits, st = dec.prefill_batch(PROMPTS, base_dtype=torch.float32, wkv_chunked=True)
    assert _lib.counters()["seq_chunked"] - n0 == TINY.n_layer
    step_logits, step_st = dec.prefill_batch(PROMPTS, base_dtype=torch.float32, wkv_chunked=False)
    for i, pr in enumerate(PROMPTS):
        ref, ost = X.prefill(p, W, pr, TINY.n_layer, TINY.n_head)
        e, ew = rel(ref, logits[i].cpu().numpy()), rel(ost.wkv[:, 0], st.wkv[:, i].cpu().numpy())
        print(f"[prefill] chunked WKV row {i} (T={len(pr)}): logits {e:.2e}, wkv {ew:.2e}", flush=True)
        assert e < 1e-4 and ew < 1e-4, i
        assert rel(step_logits[i].cpu().numpy(), logits[i].cpu().numpy()) < 1e-5, i
    rng = np.random.default_rng(35)
    long_prompt = [int(t) for t in rng.integers(0, TINY.vocab, 600)]
    assert wkv_chunked_prefers(1, 600, TINY.n_head)
    n0 = _lib.counters()["seq_chunked"]
    logits, st = dec.prefill_batch([long_prompt], base_dtype=torch.float32)
    assert _lib.counters()["seq_chunked"] - n0 == TINY.n_layer
    ref, ost = X.prefill(p, W, long_prompt, TINY.n_layer, TINY.n_head)
    e, ew = rel(ref, logits[0].cpu().numpy()), rel(ost.wkv[:, 0], st.wkv[:, 0].cpu().numpy())
    print(f"[prefill] chunked WKV T=600: logits {e:.2e}, wkv {ew:.2e}", flush=True)
    assert e < 1e-4 and ew < 1e-4


def test_prefill_past_65535_rows_rows_independent(tiny_model):
    """A long pass of more than 65535 rows (two prompts of 35,000 tokens: the
    many-row layer norm, the dense GEMM route, the two-part low-rank kernel,
    the time-chunked WKV): each row's logits and states equal that prompt
    prefilled alone bitwise (every kernel on this path computes a row from
    that row alone, in the same order for both launches)."""
    case("prefill fp16 base, 70,000 rows")
    proj, W = tiny_model
    p = syn.x070_dense_params(TINY, seed=36, lora_dtype=np.float16)
    dec = X070Decoder(TINY.n_layer, TINY.n_embd, TINY.ffn, TINY.vocab, p, proj, DEV)
    rng = np.random.default_rng(36)
    prompts = [[int(t) for t in rng.integers(0, TINY.vocab, 35000)] for _ in range(2)]
    logits, st = dec.prefill_batch(prompts, base_dtype=torch.float16)
    assert torch.isfinite(logits).all()
    for i, pr in enumerate(prompts):
        alone, st1 = dec.prefill_batch([pr], base_dtype=torch.float16)
        assert torch.equal(alone[0], logits[i]), i
        assert torch.equal(st1.wkv[:, 0], st.wkv[:, i]), i


def test_prefill_then_decode_continues_the_prompt(tiny_model):
    """The state a parallel prefill leaves continues by decode steps exactly
    as decoding the prompt token by token does (fp32 base, 1e-4)."""
    case("prefill then decode")
    proj, W = tiny_model
    p = syn.x070_dense_params(TINY, seed=33, lora_dtype=np.float32)
    dec = X070Decoder(TINY.n_layer, TINY.n_embd, TINY.ffn, TINY.vocab, p, proj, DEV)
    logits, st = dec.prefill_batch(PROMPTS[:2], base_dtype=torch.float32)
    osts = []
    for pr in PROMPTS[:2]:
        o = X.State.zeros(TINY.n_layer, 1, TINY.n_head)
        for tok in pr:
            X.step(p, W, [tok], o, TINY.n_layer, TINY.n_head)
        osts.append(o)
    for step_ids in ([3, 4], [100, 200], [7, 7]):
        got = dec.step_batch(step_ids, st).cpu().numpy()
        for i, o in enumerate(osts):
            ref = X.step(p, W, [step_ids[i]], o, TINY.n_layer, TINY.n_head)
            assert rel(ref, got[i]) < 1e-4, (step_ids, i)


def _states_equal(a, b):
    return all(torch.equal(x, y) for x, y in zip((a.wkv, a.tmix_prev, a.cmix_prev, a.v_first),
                                                 (b.wkv, b.tmix_prev, b.cmix_prev, b.v_first)))


@pytest.mark.parametrize("base,chunked", [(torch.float16, False), (torch.float32, True), (torch.float16, True)])
def test_prefill_graph_replays_match_eager(tiny_model, base, chunked):
    """prefill_batch(graph=True): the pass captured once per (B, T, kind) and
    replayed for other prompts of the same shape gives the eager pass's
    logits and state bitwise, every replay, with eager passes of other
    shapes (which reuse and regrow the pass buffers) in between."""
    case(f"prefill graph replays, base {base}, chunked WKV {chunked}")
    proj, W = tiny_model
    p = syn.x070_dense_params(TINY, seed=36, lora_dtype=np.float16)
    dec = X070Decoder(TINY.n_layer, TINY.n_embd, TINY.ffn, TINY.vocab, p, proj, DEV)
    rng = np.random.default_rng(36)
    T = max(len(pr) for pr in PROMPTS)
    sets = [PROMPTS] + [[[int(t) for t in rng.integers(0, TINY.vocab, n)] for n in rng.integers(1, T + 1, len(PROMPTS))]
                        for _ in range(3)]
    for pr in sets[1:]:
        pr[0] = pr[0] + [1] * (T - len(pr[0]))   # the same (B, T) for every set
    kw = dict(base_dtype=base, short_rows=0, wkv_chunked=chunked)
    for rep, pr in enumerate(sets + sets[:1]):
        eager, est = dec.prefill_batch(pr, **kw)
        torch.cuda.synchronize()
        got, gst = dec.prefill_batch(pr, graph=True, **kw)
        torch.cuda.synchronize()
        assert torch.equal(got, eager) and _states_equal(gst, est), rep
        dec.prefill_batch([pr[0] * 2, pr[1]], **kw)   # another shape between replays
        torch.cuda.synchronize()
    # the graphed rows still agree with the oracle
    ref, _ = X.prefill(p, W, sets[0][3], TINY.n_layer, TINY.n_head, f16_base=base == torch.float16)
    got, _ = dec.prefill_batch(sets[0], graph=True, **kw)
    assert rel(ref, got[3].cpu().numpy()) < (2e-3 if base == torch.float16 else 1e-4)


def _mixed_projections(shape, seed=61):
    """A model whose projections take every long-pass layout of the matrix
    cores: r/k/v sym 8-bit (one fused group), o_proj sb6 5-bit, ffn key sym
    6-bit, ffn value sb6 6-bit, head sym 8-bit.  Returns (key → Proj on the
    device, key → fp64 dense weight of the oracle)."""
    from oracle import oracle as O
    from swiftrwkv_amd.x070 import Proj
    rng = np.random.default_rng(seed)
    proj, W = {}, {}
    for key, OUT, IN in shape.projections():
        w = (rng.standard_normal((OUT, IN)) * 0.02).astype(np.float32)
        if ".att.output." in key or ".ffn.value." in key:
            bits = 5 if ".att.output." in key else 6
            disk = Q.encode_sb6(w, bits, 8)
            qblk, qsqm, ddm, xb = Q.rwkvq_sb6_to_k3(disk["codes_packed"], disk["gw_qsqm"], disk["gw_d"], disk["gw_dm"],
                                                    disk.get("gw_qh"), disk.get("gw_qh2"), (OUT, IN))
            assert xb == bits - 4
            proj[key] = Proj("sb6", (dev(qblk), dev(qsqm), dev(ddm.view(np.float16))), OUT, IN, bits=bits, xbits=xb)
            W[key] = O.sb6_dequant(qblk, qsqm, ddm.view(np.uint16), OUT, IN, xb).astype(np.float64)
        else:
            bits = 6 if ".ffn.key." in key else 8
            disk = Q.encode_sym(w, bits, 8)
            qblk = (disk["codes"].view(np.uint8) if bits == 8 else
                    Q.rwkvq_sym_interleave(disk["codes_packed"], disk["gw_qh"], disk["gw_qh2"], (OUT, IN)))
            qs, d = disk["gw_qs"].view(np.uint8), disk["gw_d"]
            proj[key] = Proj("sym", (dev(qblk), dev(qs), dev(d)), OUT, IN, bits=bits)
            W[key] = O.sym_dequant(qblk, qs, d.view(np.uint16), OUT, IN, bits).astype(np.float64)
    return proj, W


def test_prefill_fp16_base_sym_and_wide_sb6_layouts():
    """The fp16 long pass of a model on the sym 8 / 6-bit and sb6 5 / 6-bit
    layouts (the r/k/v group as one sym launch) against the oracle's parallel
    pass with the same fp16 rounding points; every projection on the matrix
    cores (launch counters), none through a dense weight."""
    case("prefill fp16 base, sym + 5/6-bit sb6 model")
    from swiftrwkv_amd import _lib
    proj, W = _mixed_projections(TINY)
    p = syn.x070_dense_params(TINY, seed=62, lora_dtype=np.float16)
    dec = X070Decoder(TINY.n_layer, TINY.n_embd, TINY.ffn, TINY.vocab, p, proj, DEV)
    assert dec.proj["blocks.0.att.rkv"].kind == "sym" and dec.proj["blocks.0.att.rkv"].out_per == TINY.n_embd
    c0 = _lib.counters()
    logits, st = dec.prefill_batch(PROMPTS, base_dtype=torch.float16, short_rows=0)
    c1 = _lib.counters()
    assert c1["sym_gemm"] - c0["sym_gemm"] == 2 * TINY.n_layer      # r/k/v group, ffn key
    assert c1["sb6_gemm"] - c0["sb6_gemm"] == 2 * TINY.n_layer      # o_proj, ffn value
    assert c1["sym_dequant"] == c0["sym_dequant"] and c1["sb6_dequant"] == c0["sb6_dequant"]
    for i, pr in enumerate(PROMPTS):
        ref, ost = X.prefill(p, W, pr, TINY.n_layer, TINY.n_head, f16_base=True)
        e = rel(ref, logits[i].cpu().numpy())
        ew = rel(ost.wkv[:, 0], st.wkv[:, i].cpu().numpy())
        print(f"[prefill] sym/sb6 5-6 bit row {i} (T={len(pr)}): logits {e:.2e}, wkv {ew:.2e}", flush=True)
        assert e < 2e-3 and ew < 2e-3, i


def test_prefill_0b4_width_fp16_base(orc):
    """The 0.4B width (n_embd 1024, FFN 4096, H 16; four layers sharing
    packed bytes, the 65536-row head), four prompts of 7..64 tokens on the
    fp16 long pass, against the oracle with its rounding points."""
    case("prefill 0.4B width, fp16 base")
    shape = syn.X070Shape("0.4B width, 4 layers", 4, 1024, 4096)
    proj = syn.x070_projections(shape, nthreads=16, share_layers=True)
    memo, W = {}, {}
    for k, q in proj.items():
        if id(q[0]) not in memo:
            memo[id(q[0])] = X.dequant_projections({k: q})[k]
        W[k] = memo[id(q[0])]
    p = syn.x070_dense_params(shape, seed=34, lora_dtype=np.float16)
    dec = X070Decoder(shape.n_layer, shape.n_embd, shape.ffn, shape.vocab, p, proj, DEV)
    rng = np.random.default_rng(34)
    prompts = [list(rng.integers(0, shape.vocab, n)) for n in (64, 7, 33, 50)]
    logits, _ = dec.prefill_batch(prompts, base_dtype=torch.float16, short_rows=0)
    for i, pr in enumerate(prompts):
        ref, _ = X.prefill(p, W, pr, shape.n_layer, shape.n_head, f16_base=True)
        e = rel(ref, logits[i].cpu().numpy())
        print(f"[prefill] 0.4B width fp16 base row {i} (T={len(pr)}): logits {e:.2e}", flush=True)
        assert e < 2e-3, i
