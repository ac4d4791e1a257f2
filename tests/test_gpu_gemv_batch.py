"""GPU parity of the matrix-core batched sb6 GEMV (rwkv_sb6_gemv_batch):
every row within fp32 rounding of the one-input VALU GEMV on that row alone
(max|batch − single| / max|single| ≤ 1e-5, the batch-vs-single bound of
BatchGenerateTests.swift:56,61), and against the fp64 oracle at the GEMV
bound (2e-5, RwkvqSb6GEMVTests.swift:53-77); fused groups and epilogues."""
import sys

import numpy as np
import pytest
import torch

from swiftrwkv_amd import _lib, quant as Q
from tests.test_gpu_model_shapes import random_k3

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def host(t):
    return t.detach().float().cpu().numpy()


def rel(ref, got):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(ref - np.asarray(got, np.float64)).max() / (np.abs(ref).max() + 1e-30))


def singles(x, w, OUT, IN, out_per=None):
    """Each input row alone through the one-input GEMV."""
    K = 1 if out_per is None else OUT // out_per
    N = x.shape[0] // K
    return torch.cat([Q.rwkvq_sb6_gemv(x[n * K:(n + 1) * K], *w, OUT, IN, 0, out_per=out_per) for n in range(N)])


SHAPES = [(768, 768), (3072, 768), (768, 3072), (2048, 2048), (1024, 4096), (4096, 1024), (65536, 768),
          (4096, 4096), (14336, 4096), (4096, 14336)]


@pytest.mark.parametrize("OUT,IN", SHAPES)
@pytest.mark.parametrize("N", [2, 8, 16, 17, 32])
def test_batch_matches_single_rows_and_oracle(orc, OUT, IN, N):
    case(f"sb6 batched gemv {OUT}x{IN} N={N}")
    rng = np.random.default_rng(OUT + 3 * IN + N)
    qblk, qsqm, ddm = random_k3(OUT, IN, rng)
    w = (dev(qblk), dev(qsqm), dev(ddm))
    x = rng.standard_normal((N, IN)).astype(np.float32)
    xd = dev(x)
    assert Q.rwkvq_sb6_gemv_batch_applies(N, OUT, IN, 0)
    y = Q.rwkvq_sb6_gemv_batch(xd, *w, OUT, IN)
    ys = singles(xd, w, OUT, IN)
    got, one = host(y), host(ys)
    worst = max(rel(one[n], got[n]) for n in range(N))
    print(f"[gemv batch] {OUT}x{IN} N={N}: rel to single rows {worst:.2e}", flush=True)
    assert worst < 1e-5
    if OUT * IN <= 4096 * 4096 or N == 2:
        want = orc.sb6_gemv_f64(x, qblk, qsqm, ddm.view(np.uint16), OUT, IN, 0)
        assert rel(want, got) < 2e-5


@pytest.mark.parametrize("D,N", [(768, 8), (1024, 32), (4096, 16)])
def test_fused_group_and_epilogues(orc, D, N):
    """r/k/v of one layer as a row-concatenated group (row o of input n reads
    x[3n + o/D]); the add and relu² epilogues against the one-input kernel's."""
    case(f"sb6 batched gemv fused 3x{D}x{D} N={N}, epilogues")
    rng = np.random.default_rng(D + N)
    qblk, qsqm, ddm = random_k3(3 * D, D, rng)
    w = (dev(qblk), dev(qsqm), dev(ddm))
    x = dev(rng.standard_normal((3 * N, D)).astype(np.float32))
    y = Q.rwkvq_sb6_gemv_batch(x, *w, 3 * D, D, out_per=D)
    ys = singles(x, w, 3 * D, D, out_per=D)
    assert rel(host(ys), host(y)) < 1e-5
    # epilogues on one matrix
    q1 = (w[0][:D], w[1][:D], w[2][:D])
    xm = dev(rng.standard_normal((N, D)).astype(np.float32))
    base = dev(rng.standard_normal((N, D)).astype(np.float32))
    y_add = Q.rwkvq_sb6_gemv_batch(xm, *q1, D, D, epilogue="add", out=base.clone())
    single = singles(xm, q1, D, D)
    assert rel(host(base + single), host(y_add)) < 1e-5
    y_r2 = Q.rwkvq_sb6_gemv_batch(xm, *q1, D, D, epilogue="relu2")
    assert rel(host(torch.relu(single) ** 2), host(y_r2)) < 2e-5


def t16_unpack(tq, ts, tm, OUT, IN):
    """T16 → (K3 code bytes [OUT, NU·16], s [OUT, NU] fp16, m [OUT, NU] fp32),
    the inverse of the layout rwkv_sb6_t16_pack documents: per (16-row tile,
    4-unit group) 1 KiB of codes whose 16 bytes at (g·16 + i)·16 are dword g
    of units 4G..4G+3 of row 16r + i; s [16 rows][4 units]; m [16 rows]
    [4 high, 4 low] bf16 parts."""
    NU, NG = IN // 32, IN // 128
    d = tq.view(np.uint32).reshape(OUT // 16, NG, 4, 16, 4)           # [r][G][dword g][row i][unit k]
    q = d.transpose(0, 3, 1, 4, 2).reshape(OUT, NU, 4).view(np.uint8).reshape(OUT, NU * 16)
    sc = ts.reshape(OUT // 16, NG, 16, 4).transpose(0, 2, 1, 3).reshape(OUT, NU)
    mb = tm.reshape(OUT // 16, NG, 16, 2, 4).astype(np.float32)       # [r][G][row][hi/lo][unit]
    mc = (mb[:, :, :, 0, :] + mb[:, :, :, 1, :]).transpose(0, 2, 1, 3).reshape(OUT, NU)
    return q, sc, mc


@pytest.mark.parametrize("OUT,IN", [(768, 768), (192, 2048), (4096, 1024)])
def test_t16_pack_is_the_k3_weights(orc, OUT, IN):
    """rwkv_sb6_t16_pack: the codes are the K3 bytes permuted, and code·s + m
    from its scales is bitwise the oracle's dequantised weight (w = code·s + m,
    s = half(qs·d), m = half(qm·dm), RwkvqDequant.swift:116-140) everywhere."""
    case(f"sb6 T16 pack {OUT}x{IN}")
    rng = np.random.default_rng(OUT + IN)
    qblk, qsqm, ddm = random_k3(OUT, IN, rng)
    tq, ts, tm = Q.rwkvq_sb6_t16(dev(qblk), dev(qsqm), dev(ddm), OUT, IN)
    q, sc, mc = t16_unpack(tq.cpu().numpy(), ts.cpu().numpy(), tm.float().cpu().numpy(), OUT, IN)
    assert np.array_equal(q, qblk)
    codes = np.empty((OUT, IN), np.float32)
    qb = qblk.reshape(OUT, IN // 32, 16)
    codes.reshape(OUT, IN // 32, 32)[..., :16] = qb & 0xF
    codes.reshape(OUT, IN // 32, 32)[..., 16:] = qb >> 4
    w = codes * np.repeat(sc.astype(np.float32), 32, axis=1) + np.repeat(mc, 32, axis=1)
    want = orc.sb6_dequant(qblk, qsqm, ddm.view(np.uint16), OUT, IN, 0)
    assert np.array_equal(w.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("OUT,IN", [(768, 768), (3072, 768), (768, 3072), (4096, 4096), (14336, 4096),
                                    (4096, 14336), (65536, 768)])
@pytest.mark.parametrize("N", [2, 16, 17, 32])
def test_t16_batch_matches_k3_batch_and_oracle(orc, OUT, IN, N):
    case(f"sb6 batched gemv T16 {OUT}x{IN} N={N}")
    rng = np.random.default_rng(7 * OUT + IN + N)
    qblk, qsqm, ddm = random_k3(OUT, IN, rng)
    w = (dev(qblk), dev(qsqm), dev(ddm))
    t = Q.rwkvq_sb6_t16(*w, OUT, IN)
    x = rng.standard_normal((N, IN)).astype(np.float32)
    xd = dev(x)
    y16 = host(Q.rwkvq_sb6_gemv_batch_t16(xd, *t, OUT, IN))
    yk3 = host(Q.rwkvq_sb6_gemv_batch(xd, *w, OUT, IN))
    worst = max(rel(yk3[n], y16[n]) for n in range(N))
    print(f"[gemv batch t16] {OUT}x{IN} N={N}: rel to the K3 batch kernel {worst:.2e}", flush=True)
    assert worst < 1e-5
    if OUT * IN <= 4096 * 4096 or N == 2:
        want = orc.sb6_gemv_f64(x, qblk, qsqm, ddm.view(np.uint16), OUT, IN, 0)
        assert rel(want, y16) < 2e-5


@pytest.mark.parametrize("D,N", [(768, 8), (4096, 16)])
def test_t16_fused_group_and_epilogues(D, N):
    case(f"sb6 batched gemv T16 fused 3x{D}x{D} N={N}, epilogues")
    rng = np.random.default_rng(3 * D + N)
    qblk, qsqm, ddm = random_k3(3 * D, D, rng)
    w = (dev(qblk), dev(qsqm), dev(ddm))
    t = Q.rwkvq_sb6_t16(*w, 3 * D, D)
    x = dev(rng.standard_normal((3 * N, D)).astype(np.float32))
    y = Q.rwkvq_sb6_gemv_batch_t16(x, *t, 3 * D, D, out_per=D)
    ys = singles(x, w, 3 * D, D, out_per=D)
    assert rel(host(ys), host(y)) < 1e-5
    t1 = Q.rwkvq_sb6_t16(w[0][:D], w[1][:D], w[2][:D], D, D)
    xm = dev(rng.standard_normal((N, D)).astype(np.float32))
    base = dev(rng.standard_normal((N, D)).astype(np.float32))
    single = singles(xm, (w[0][:D], w[1][:D], w[2][:D]), D, D)
    y_add = Q.rwkvq_sb6_gemv_batch_t16(xm, *t1, D, D, epilogue="add", out=base.clone())
    assert rel(host(base + single), host(y_add)) < 1e-5
    y_r2 = Q.rwkvq_sb6_gemv_batch_t16(xm, *t1, D, D, epilogue="relu2")
    assert rel(host(torch.relu(single) ** 2), host(y_r2)) < 2e-5
    a = Q.rwkvq_sb6_gemv_batch_t16(xm, *t1, D, D)
    b = Q.rwkvq_sb6_gemv_batch_t16(xm, *t1, D, D)
    assert torch.equal(a, b)


# K of 2 unit groups (two of four waves idle), 6 (waves with 2 and 1), 8, 16,
# 24 (3: an odd count) and 32 per 16-row tile; one, two (3072, 4096 and 8192
# rows) and four (8192 rows at 17+ inputs) row tiles per workgroup; past
# K = 4096 the looping waves (8 and 5 unit groups each, the 4608-row matrix in
# row-tile pairs); K of 2 and 4 unit groups with four row tiles per workgroup
# (8192x256 at 17+ inputs, 16384x512)
@pytest.mark.parametrize("OUT,IN", [(64, 256), (768, 768), (3072, 768), (768, 3072), (1024, 1024), (4096, 1024),
                                    (1024, 4096), (192, 2048), (8192, 768), (256, 8192), (4608, 5120),
                                    (8192, 256), (16384, 512)])
@pytest.mark.parametrize("N", [2, 8, 16, 17, 32])
def test_t16_rows_kernel_matches_single_rows_and_oracle(orc, OUT, IN, N):
    case(f"sb6 batched gemv T16 row-owned {OUT}x{IN} N={N}")
    rng = np.random.default_rng(11 * OUT + IN + N)
    qblk, qsqm, ddm = random_k3(OUT, IN, rng)
    w = (dev(qblk), dev(qsqm), dev(ddm))
    t = Q.rwkvq_sb6_t16(*w, OUT, IN)
    x = rng.standard_normal((N, IN)).astype(np.float32)
    xd = dev(x)
    yr = host(Q.rwkvq_sb6_gemv_batch_t16(xd, *t, OUT, IN, rows_kernel=True))
    one = host(singles(xd, w, OUT, IN))
    worst = max(rel(one[n], yr[n]) for n in range(N))
    print(f"[gemv batch t16 rows] {OUT}x{IN} N={N}: rel to the one-input kernel {worst:.2e}", flush=True)
    assert worst < 1e-5
    want = orc.sb6_gemv_f64(x, qblk, qsqm, ddm.view(np.uint16), OUT, IN, 0)
    assert rel(want, yr) < 2e-5


@pytest.mark.parametrize("D,N", [(768, 8), (1024, 32)])
def test_t16_rows_kernel_fused_group_and_epilogues(D, N):
    case(f"sb6 batched gemv T16 row-owned fused 3x{D}x{D} N={N}, epilogues")
    rng = np.random.default_rng(5 * D + N)
    qblk, qsqm, ddm = random_k3(3 * D, D, rng)
    w = (dev(qblk), dev(qsqm), dev(ddm))
    t = Q.rwkvq_sb6_t16(*w, 3 * D, D)
    x = dev(rng.standard_normal((3 * N, D)).astype(np.float32))
    y = Q.rwkvq_sb6_gemv_batch_t16(x, *t, 3 * D, D, out_per=D, rows_kernel=True)
    assert rel(host(singles(x, w, 3 * D, D, out_per=D)), host(y)) < 1e-5
    t1 = Q.rwkvq_sb6_t16(w[0][:D], w[1][:D], w[2][:D], D, D)
    xm = dev(rng.standard_normal((N, D)).astype(np.float32))
    base = dev(rng.standard_normal((N, D)).astype(np.float32))
    single = singles(xm, (w[0][:D], w[1][:D], w[2][:D]), D, D)
    y_add = Q.rwkvq_sb6_gemv_batch_t16(xm, *t1, D, D, epilogue="add", out=base.clone(), rows_kernel=True)
    assert rel(host(base + single), host(y_add)) < 1e-5
    y_r2 = Q.rwkvq_sb6_gemv_batch_t16(xm, *t1, D, D, epilogue="relu2", rows_kernel=True)
    assert rel(host(torch.relu(single) ** 2), host(y_r2)) < 2e-5
    a = Q.rwkvq_sb6_gemv_batch_t16(xm, *t1, D, D, rows_kernel=True)
    b = Q.rwkvq_sb6_gemv_batch_t16(xm, *t1, D, D, rows_kernel=True)
    assert torch.equal(a, b)
    # rows of other inputs untouched: the kernel stores inputs < N only
    out = torch.full((N, D), 7.0, device=DEV)
    Q.rwkvq_sb6_gemv_batch_t16(xm[:N - 1].contiguous(), *t1, D, D, out=out[:N - 1], rows_kernel=True)
    assert torch.all(out[N - 1] == 7.0)


def test_contract_and_declines():
    case("sb6 batched gemv: applicability, workspace, counters")
    L = _lib.lib()
    assert L.rwkv_sb6_gemv_batch_applies(8, 768, 768, 0, 768) == 1
    assert L.rwkv_sb6_gemv_batch_applies(1, 768, 768, 0, 768) == 0      # one row: the VALU kernel
    assert L.rwkv_sb6_gemv_batch_applies(33, 768, 768, 0, 768) == 0     # more: split the batch
    assert L.rwkv_sb6_gemv_batch_applies(8, 768, 768, 1, 768) == 0      # wider codes
    assert L.rwkv_sb6_gemv_batch_applies(8, 768, 800, 0, 768) == 0      # IN % 256
    assert L.rwkv_sb6_gemv_batch_applies(8, 96, 768, 0, 96) == 0        # out_per % 64
    rng = np.random.default_rng(5)
    qblk, qsqm, ddm = (dev(z) for z in random_k3(768, 768, rng))
    x = dev(rng.standard_normal((8, 768)).astype(np.float32))
    need = L.rwkv_sb6_gemv_batch_workspace(8, 768, 768, 768)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    y = torch.empty((8, 768), device=DEV)
    before = _lib.counters()["sb6_batch"]
    st = L.rwkv_sb6_gemv_batch(x.data_ptr(), 8, qblk.data_ptr(), qsqm.data_ptr(), ddm.data_ptr(), y.data_ptr(),
                               768, 768, 0, 768, 0, ws.data_ptr(), need - 4, None)
    assert st != 0 and b"workspace" in L.rwkv_last_error()
    assert _lib.counters()["sb6_batch"] == before
    Q.rwkvq_sb6_gemv_batch(x, qblk, qsqm, ddm, 768, 768, workspace=ws)
    assert _lib.counters()["sb6_batch"] == before + 1
    # deterministic: the same call twice gives the same bits
    a = Q.rwkvq_sb6_gemv_batch(x, qblk, qsqm, ddm, 768, 768, workspace=ws)
    b = Q.rwkvq_sb6_gemv_batch(x, qblk, qsqm, ddm, 768, 768, workspace=ws)
    assert torch.equal(a, b)


def test_decoder_batch_rows_match_each_row_alone():
    """X070Decoder.step_batch with 9 and 24 rows (the batched matrix-core GEMV
    for every sb6 projection) against each row stepped alone (the one-input
    kernels): logits and states within fp32 rounding over three tokens."""
    from swiftrwkv_amd import synthetic as syn
    from swiftrwkv_amd.x070 import X070Decoder
    tiny = syn.X070Shape("tiny", 2, 256, 1024, vocab=512)
    p = syn.x070_dense_params(tiny, seed=13, lora_dtype=np.float32)
    proj = syn.x070_projections(tiny, nthreads=4)
    dec = X070Decoder(tiny.n_layer, tiny.n_embd, tiny.ffn, tiny.vocab, p, proj, DEV)
    dec.batch_mfma = True   # the matrix-core path for every projection, whatever the size rule
    rng = np.random.default_rng(13)
    assert dec._batch_chunks(dec.proj["head.weight"], 40) == [20, 20]
    for N in (9, 24):
        case(f"x070 step_batch N={N} vs rows alone")
        st = dec.new_state(N)
        alone = [dec.new_state(1) for _ in range(N)]
        for t in range(3):
            ids = rng.integers(0, tiny.vocab, N).tolist()
            before = _lib.counters()["sb6_batch"]
            got = host(dec.step_batch(ids, st))
            assert _lib.counters()["sb6_batch"] - before == 4 * tiny.n_layer + 1   # r/k/v, o, key, value; head
            for n in range(N):
                one = host(dec.step_batch([ids[n]], alone[n]))[0]
                e = rel(one, got[n])
                assert e < 1e-5, (N, t, n, e)
        for n in range(N):
            assert rel(host(alone[n].wkv[:, 0]), host(st.wkv[:, n])) < 1e-5
