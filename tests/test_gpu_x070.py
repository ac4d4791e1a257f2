"""GPU parity of the x070 decode step around the hot path (layer norms, token
shift, low-rank branches, tmix core, GEMV epilogues, whole steps) against the
fp64 oracle (oracle/x070.py), through the C ABI.

Tolerances (max|got − ref| / max|ref| unless stated): 1e-5 for the fp32
elementwise kernels (layer norm, lerps); one fp16 ulp (2^-10 relative per
element) for the low-rank products, whose fp16 rounding of an fp32 sum may
land on the other side of a rounding boundary than the fp64 sum; 1e-4 for the
tmix core and whole decode steps (the WKV bound of 1e-5 per step with those
fp16 roundings upstream).  GEMV epilogues are bitwise the plain GEMV followed by
the separate operations.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import x070 as X
from swiftrwkv_amd import _lib, synthetic as syn
from swiftrwkv_amd.x070 import X070Decoder, LN_EPS

pytestmark = pytest.mark.gpu
DEV = "cuda"
TINY = syn.X070Shape("tiny", 2, 256, 1024, vocab=512)


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def rel(ref, got):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(ref - np.asarray(got, np.float64)).max() / (np.abs(ref).max() + 1e-30))


@pytest.fixture(scope="module")
def tiny():
    p = syn.x070_dense_params(TINY, seed=3)
    proj = syn.x070_projections(TINY, nthreads=4)
    return p, proj, X.dequant_projections(proj)


@pytest.fixture(scope="module")
def decoder(tiny):
    p, proj, _ = tiny
    return X070Decoder(TINY.n_layer, TINY.n_embd, TINY.ffn, TINY.vocab, p, proj, DEV)


@pytest.mark.parametrize("D", [256, 768, 4096])
def test_layer_norm(D):
    case(f"layer_norm D={D}")
    rng = np.random.default_rng(D)
    x = (rng.standard_normal((5, D)) * 2 + 0.5).astype(np.float32)
    w, b = rng.standard_normal(D).astype(np.float32), rng.standard_normal(D).astype(np.float32)
    y = torch.empty((5, D), device=DEV)
    xd, wd, bd = dev(x), dev(w), dev(b)   # alive across the launch
    _lib.call("rwkv_layer_norm", xd.data_ptr(), _lib.F32, None, 0, wd.data_ptr(), bd.data_ptr(),
              y.data_ptr(), 5, D, LN_EPS, None)
    torch.cuda.synchronize()
    assert rel(X.layer_norm(x, w, b), y.cpu().numpy()) < 1e-5


def test_layer_norm_gather_f16_table_and_bad_ids():
    case("layer_norm gather")
    rng = np.random.default_rng(1)
    V, D = 300, 768
    tab = (rng.standard_normal((V, D)) * 0.5).astype(np.float16)
    w, b = rng.standard_normal(D).astype(np.float32), rng.standard_normal(D).astype(np.float32)
    ids = np.array([5, 299, -1, 0, 300], np.int32)
    y = torch.empty((5, D), device=DEV)
    td, idd, wd, bd = dev(tab), dev(ids), dev(w), dev(b)
    _lib.call("rwkv_layer_norm", td.data_ptr(), _lib.F16, idd.data_ptr(), V, wd.data_ptr(),
              bd.data_ptr(), y.data_ptr(), 5, D, LN_EPS, None)
    got = y.cpu().numpy()
    good = [0, 1, 3]
    assert rel(X.layer_norm(tab.astype(np.float64)[ids[good]], w, b), got[good]) < 1e-5
    assert np.isnan(got[[2, 4]]).all()
    _lib.call("rwkv_layer_norm", None, _lib.F32, None, 0, None, None, None, 0, D, LN_EPS, None)   # N = 0: no-op


@pytest.mark.parametrize("D", [768, 4096, 8192])
def test_layer_norm_many_rows_bitwise(D):
    """From 1024 rows rwkv_layer_norm takes one wave per row: every row equals
    the row of a short launch bitwise (rows are independent), within 1e-5 of
    the oracle; a gather with ids outside the table gives NaN rows."""
    case(f"layer_norm many rows D={D}")
    rng = np.random.default_rng(D + 1)
    N = 1030

    def ln(xd, dt, ids, rows, n):
        y = torch.empty((n, D), device=DEV)
        _lib.call("rwkv_layer_norm", xd.data_ptr(), dt, None if ids is None else ids.data_ptr(), rows, wd.data_ptr(),
                  bd.data_ptr(), y.data_ptr(), n, D, LN_EPS, None)
        return y

    x = (rng.standard_normal((N, D)) * 2 + 0.5).astype(np.float32)
    w, b = rng.standard_normal(D).astype(np.float32), rng.standard_normal(D).astype(np.float32)
    xd, wd, bd = dev(x), dev(w), dev(b)
    y = ln(xd, _lib.F32, None, 0, N)
    for lo in (0, N - 300):
        assert torch.equal(y[lo:lo + 300], ln(xd[lo:lo + 300].contiguous(), _lib.F32, None, 0, 300))
    rows = [0, 1, 517, N - 1]
    assert rel(X.layer_norm(x[rows], w, b), y[rows].cpu().numpy()) < 1e-5
    V = 40
    tab = (rng.standard_normal((V, D)) * 0.5).astype(np.float16)
    ids = rng.integers(0, V, N).astype(np.int32)
    ids[[3, 700]] = [-1, V]
    td, idd = dev(tab), dev(ids)
    g = ln(td, _lib.F16, idd, V, N).cpu().numpy()
    assert np.isnan(g[[3, 700]]).all()
    good = np.setdiff1d(np.arange(N), [3, 700])
    short = ln(td, _lib.F16, dev(ids[good[:200]].copy()), V, 200).cpu().numpy()
    assert np.array_equal(short, g[good[:200]])


@pytest.mark.parametrize("nc", [6, 1])
def test_shift_mix(nc):
    case(f"shift_mix nc={nc}")
    rng = np.random.default_rng(nc)
    N, D = 3, 768
    x = rng.standard_normal((N, D)).astype(np.float32)
    w, b = rng.standard_normal(D).astype(np.float32), rng.standard_normal(D).astype(np.float32)
    prev = rng.standard_normal((N, D)).astype(np.float32)
    coef = rng.uniform(0, 1, (nc, D)).astype(np.float32)
    prev_d = dev(prev)
    out0 = torch.empty((N, min(nc, 3), D), device=DEV)
    out1 = torch.empty((N, 4, D), device=DEV) if nc == 6 else None
    xd, wd, bd, cd = dev(x), dev(w), dev(b), dev(coef)
    _lib.call("rwkv_x070_shift_mix", xd.data_ptr(), wd.data_ptr(), bd.data_ptr(), prev_d.data_ptr(),
              cd.data_ptr(), nc, out0.data_ptr(), out1.data_ptr() if out1 is not None else None, N, D, LN_EPS,
              None)
    xl = X.layer_norm(x, w, b)
    mix, new_prev = X.shift_mix(xl, prev, list(coef))
    assert rel(new_prev, prev_d.cpu().numpy()) < 1e-5
    # coefficients r, k, v, w, a, g: out0 ← (r, k, v), out1 ← (w, a, v, g)
    got = out0.cpu().numpy()
    for c in range(min(nc, 3)):
        assert rel(mix[c], got[:, c]) < 1e-5, c
    if nc == 6:
        g1 = out1.cpu().numpy()
        for slot, c in enumerate((3, 4, 2, 5)):
            assert rel(mix[c], g1[:, slot]) < 1e-5, (slot, c)


def _fp16_ulp_close(ref, got):
    ref, got = np.asarray(ref, np.float64), np.asarray(got, np.float64)
    return np.abs(ref - got) <= 2.0 ** -10 * np.abs(ref) + 1e-6


@pytest.mark.parametrize("l", [0, 1])
@pytest.mark.parametrize("wdt", [np.float16, np.float32])
def test_lora_in(tiny, l, wdt):
    case(f"lora_in layer={l} dtype={wdt.__name__}")
    p, _, _ = tiny
    p = dict(p)
    t = f"blocks.{l}.tmix."
    for nm in "wavg":
        p[t + nm + "_lora_A.weight"] = p[t + nm + "_lora_A.weight"].astype(wdt)
    rng = np.random.default_rng(l)
    N, D = 2, TINY.n_embd
    xmix = rng.standard_normal((N, 4, D)).astype(np.float32)   # w, a, v, g inputs
    rw, ra, rv, rg = syn.lora_ranks(D)
    wcat = np.concatenate([p[t + nm + "_lora_A.weight"] for nm in "wavg"])
    la = torch.full((N, rw + ra + rv + rg), 7.0, device=DEV)
    xm_d, wc_d = dev(xmix), dev(wcat)
    _lib.call("rwkv_x070_lora_in", xm_d.data_ptr(), wc_d.data_ptr(), _lib.F16 if wdt == np.float16 else _lib.F32,
              rw, ra, rv, rg, int(l > 0), la.data_ptr(), N, D, None)
    got = la.cpu().numpy()
    ref = X.lora_in(p, l, xmix[:, 0], xmix[:, 1], xmix[:, 2], xmix[:, 3])
    offs = np.cumsum([0, rw, ra, rv, rg])
    for i, r in enumerate(ref):
        g = got[:, offs[i]:offs[i + 1]]
        if r is None:
            assert (g == 7.0).all()   # layer 0: the v branch is not computed
        elif wdt == np.float16:
            assert _fp16_ulp_close(r, g).all(), i
        else:
            assert rel(r, g) < 1e-5, i


@pytest.mark.parametrize("l", [0, 1])
@pytest.mark.parametrize("N", [1, 5, 64])   # 64 rows x 4 heads: the sixteen-rows-per-wave layout
def test_tmix_core(tiny, l, N):
    case(f"tmix_core layer={l} N={N}")
    p, _, _ = tiny
    D, H = TINY.n_embd, TINY.n_head
    rw, ra, rv, rg = syn.lora_ranks(D)
    rng = np.random.default_rng(10 * l + N)
    r, k0, v0 = (rng.standard_normal((N, D)).astype(np.float32) for _ in range(3))
    la = [X.f16r(rng.standard_normal((N, n))).astype(np.float32) for n in (rw, ra, rv, rg)]
    la[0] = np.tanh(la[0]).astype(np.float32)
    v_first = rng.standard_normal((N, D)).astype(np.float32)
    wkv = (rng.standard_normal((N, H, 64, 64)) * 0.1).astype(np.float32)
    t = f"blocks.{l}.tmix."
    B = [dev(p[t + nm + "_lora_B.weight"]) for nm in "wavg"]
    bias = [dev(p[t + nm + "_lora_B.bias"].astype(np.float32)) for nm in "wav"]
    vec = {k: dev(p[t + k].astype(np.float32)) for k in ("k_k", "k_a", "r_k", "ln_x.weight", "ln_x.bias")}
    y_rkv = dev(np.concatenate([r, k0, v0], 1))
    la_d = dev(np.concatenate(la, 1))
    vf_d, st_d = dev(v_first), dev(wkv)
    out = torch.empty((N, D), device=DEV)
    _lib.call("rwkv_x070_tmix_core", y_rkv.data_ptr(), la_d.data_ptr(), *[b.data_ptr() for b in B], _lib.F16,
              rw, ra, rv, rg, *[b.data_ptr() for b in bias], vec["k_k"].data_ptr(), vec["k_a"].data_ptr(),
              vec["r_k"].data_ptr(), vec["ln_x.weight"].data_ptr(), vec["ln_x.bias"].data_ptr(), vf_d.data_ptr(),
              int(l == 0), st_d.data_ptr(), out.data_ptr(), N, H, 64e-5, None, None, None)
    tail, wkv_ref, vf_ref = X.core(p, l, r.astype(np.float64), k0.astype(np.float64), v0.astype(np.float64),
                                   [z.astype(np.float64) for z in la], v_first.astype(np.float64),
                                   wkv.astype(np.float64), H)
    # an fp16 low-rank output may round to the other fp16 neighbour of the
    # fp64 sum (one fp16 ulp); 64 rows meet such flips more often than 5
    tol = 1e-4 if N < 64 else 5e-4
    assert rel(tail, out.cpu().numpy()) < tol
    assert rel(wkv_ref, st_d.cpu().numpy()) < tol
    assert rel(vf_ref, vf_d.cpu().numpy()) < 1e-6


@pytest.mark.parametrize("N", [1, 3])
def test_gemv_epilogues_bitwise(tiny, N):
    case(f"gemv epilogues N={N}")
    _, proj, _ = tiny
    qb, qs, dd, OUT, IN = proj["blocks.0.ffn.key.weight"]
    q = [dev(qb), dev(qs), dev(dd.view(np.uint16))]
    rng = np.random.default_rng(N)
    x = dev(rng.standard_normal((N, IN)).astype(np.float32))
    res = dev(rng.standard_normal((N, OUT)).astype(np.float32))
    L = _lib.lib()
    plain = torch.empty((N, OUT), device=DEV)
    _lib.check(L.rwkv_sb6_gemv(x.data_ptr(), N, *[t.data_ptr() for t in q], plain.data_ptr(), OUT, IN, 0, None))
    added = res.clone()
    _lib.check(L.rwkv_sb6_gemv_ep(x.data_ptr(), N, *[t.data_ptr() for t in q], added.data_ptr(), OUT, IN, 0, 1, None))
    sq = torch.empty((N, OUT), device=DEV)
    _lib.check(L.rwkv_sb6_gemv_ep(x.data_ptr(), N, *[t.data_ptr() for t in q], sq.data_ptr(), OUT, IN, 0, 2, None))
    torch.cuda.synchronize()
    assert torch.equal(added, res + plain)
    h = torch.relu(plain)
    assert torch.equal(sq, h * h)
    with pytest.raises(_lib.RwkvHipError):
        _lib.check(L.rwkv_sb6_gemv_ep(x.data_ptr(), N, *[t.data_ptr() for t in q], sq.data_ptr(), OUT, IN, 0, 3,
                                      None))


@pytest.mark.parametrize("N", [1, 3, 64])   # 64 rows x 4 heads: the sixteen-rows-per-wave layout
def test_decode_steps_match_oracle(tiny, decoder, N):
    case(f"decode tiny N={N}")
    p, _, W = tiny
    st = decoder.new_state(N)
    ost = X.State.zeros(TINY.n_layer, N, TINY.n_head)
    rng = np.random.default_rng(N)
    tol = 1e-4 if N < 64 else 5e-4   # fp16 low-rank rounding flips, as in test_tmix_core
    _lib.reset_counters()
    for t in range(4):
        ids = rng.integers(0, TINY.vocab, N).astype(np.int32)
        got = decoder.step(ids, st).cpu().numpy()
        ref = X.step(p, W, ids, ost, TINY.n_layer, TINY.n_head)
        assert rel(ref, got) < tol, t
    assert rel(ost.wkv, st.wkv.cpu().numpy()) < tol
    assert rel(ost.tmix_prev, st.tmix_prev.cpu().numpy()) < tol
    assert rel(ost.cmix_prev, st.cmix_prev.cpu().numpy()) < tol
    c = _lib.counters()
    Lr = TINY.n_layer
    assert c["x070"] == 4 * (2 + 4 * Lr)          # ln0 + ln_out + 4 per layer
    if decoder._batch_chunks(decoder.proj["head.weight"], N):   # batched matrix-core GEMV, chunks <= 32 rows
        assert c["sb6_batch"] == 4 * ((N + 31) // 32) * (4 * Lr + 1)
        assert c["sb6_gemv"] == 0 and c["sb6_fused"] == 0
    else:
        assert c["sb6_gemv"] == 4 * (3 * Lr + 1)      # o_proj, ffn key, ffn value, head
        assert c["sb6_fused"] == 4 * Lr               # r/k/v
    # batch 1: each layer's r/k/v GEMV and lora_in share one launch; the
    # batched matrix-core GEMV is one launch per chunk of <= 32 rows here
    # (the row-owned kernel: every K of this shape is <= 1024)
    if decoder._batch_chunks(decoder.proj["head.weight"], N):
        ch = (N + 31) // 32
        assert decoder.launches_per_token(N) == (4 + 4 * ch) * Lr + 2 + ch
    else:
        assert decoder.launches_per_token(N) == (5 if N == 1 else 8) * Lr + 3


@pytest.mark.parametrize("D,xbits,wdt", [(768, 0, np.float16), (2048, 0, np.float16), (4096, 0, np.float16),
                                          (768, 1, np.float16), (768, 0, np.float32)])
@pytest.mark.parametrize("l", [0, 1])
def test_rkv_lora_matches_separate(D, xbits, wdt, l):
    """rwkv_x070_rkv_lora against rwkv_sb6_gemv_fused + rwkv_x070_lora_in,
    bitwise: one launch at the r/k/v widths of the 0.1B, 1.5B and 7B-class
    shapes (weights-first and inputs-first GEMV plans), the two launches for
    5-bit sb6 or fp32 low-rank matrices."""
    from swiftrwkv_amd import quant as Q
    case(f"rkv_lora D={D} xbits={xbits} {wdt.__name__} layer={l}")
    rng = np.random.default_rng(D + l)
    w = (rng.standard_normal((3 * D, D), dtype=np.float32) * np.float32(0.02))
    disk = Q.encode_sb6(w, 4 + xbits, 8)
    qb, qs, dd, xb = Q.rwkvq_sb6_to_k3(disk["codes_packed"], disk["gw_qsqm"], disk["gw_d"], disk["gw_dm"],
                                       disk.get("gw_qh"), disk.get("gw_qh2"), (3 * D, D))
    assert xb == xbits
    q = [dev(qb), dev(qs), dev(np.ascontiguousarray(dd).view(np.float16))]
    rw, ra, rv, rg = syn.lora_ranks(D)
    RT = rw + ra + rv + rg
    wcat = dev((rng.standard_normal((RT, D)) * 0.05).astype(wdt))
    wcode = _lib.F16 if wdt == np.float16 else _lib.F32
    xrkv = dev(rng.standard_normal((1, 3, D)).astype(np.float32))
    xmix = dev(rng.standard_normal((1, 4, D)).astype(np.float32))
    y1, y2 = torch.full((1, 3 * D), 5.0, device=DEV), torch.full((1, 3 * D), 5.0, device=DEV)
    la1, la2 = torch.full((1, RT), 7.0, device=DEV), torch.full((1, RT), 7.0, device=DEV)
    _lib.reset_counters()
    _lib.call("rwkv_x070_rkv_lora", xrkv.data_ptr(), *[t.data_ptr() for t in q], y1.data_ptr(), 3 * D, D, xbits, D,
              xmix.data_ptr(), wcat.data_ptr(), wcode, rw, ra, rv, rg, int(l > 0), la1.data_ptr(), None)
    c = _lib.counters()
    assert c["sb6_fused"] == 1 and c["x070"] == 1
    _lib.call("rwkv_sb6_gemv_fused", xrkv.data_ptr(), 1, *[t.data_ptr() for t in q], y2.data_ptr(), 3 * D, D, xbits,
              D, None)
    _lib.call("rwkv_x070_lora_in", xmix.data_ptr(), wcat.data_ptr(), wcode, rw, ra, rv, rg, int(l > 0),
              la2.data_ptr(), 1, D, None)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert torch.equal(la1, la2)
    if l == 0:   # the v branch is left as it was
        assert (la1[:, rw + ra:rw + ra + rv] == 7.0).all()


def test_decode_fused_rkv_lora_bitwise(tiny, decoder):
    """The decoder's batch-1 step with the r/k/v GEMV and lora_in fused, and
    with the GEMV launches forming their ln / token-shift rows themselves, is
    bitwise the step with the separate launches (logits and every state row)."""
    case("decode fused rkv+lora / rows formed in the GEMVs vs separate")
    ids = [5, 300, 17]
    outs = []
    for fuse, ln in ((True, True), (True, False), (False, False)):
        decoder.fuse_rkv_lora, decoder.fuse_ln = fuse, ln
        assert decoder._ln_fused(1) == ln
        st = decoder.new_state(1)
        outs.append([decoder.step([i], st) for i in ids] + [st.wkv.clone(), st.v_first.clone(),
                                                             st.tmix_prev.clone(), st.cmix_prev.clone()])
    decoder.fuse_rkv_lora = decoder.fuse_ln = True
    for other in outs[1:]:
        for a, b in zip(outs[0], other):
            assert torch.equal(a, b)


@pytest.mark.parametrize("D", [768, 1024, 2048])
def test_rows_formed_in_gemv_launches_bitwise(D):
    """rwkv_x070_rkv_lora_ln / ffn_key_ln / ffn_value against rwkv_x070_shift_mix
    + rwkv_x070_rkv_lora / rwkv_sb6_gemv_ep at the 0.1B, 0.4B and 1.5B widths
    (the shapes rwkv_x070_ln_fused_applies takes): outputs, the LN rows handed
    on and the shift-state copy, bitwise."""
    from swiftrwkv_amd import quant as Q
    case(f"rows formed in the GEMV launches D={D}")
    rng = np.random.default_rng(D)
    F = 4 * D
    L = _lib.lib()
    assert L.rwkv_x070_ln_fused_applies(D, F, 0) == 1

    def sb6(OUT, IN):
        w = (rng.standard_normal((OUT, IN), dtype=np.float32) * np.float32(0.02))
        disk = Q.encode_sb6(w, 4, 8)
        qb, qs, dd, _ = Q.rwkvq_sb6_to_k3(disk["codes_packed"], disk["gw_qsqm"], disk["gw_d"], disk["gw_dm"], None,
                                          None, (OUT, IN))
        return [dev(qb), dev(qs), dev(np.ascontiguousarray(dd).view(np.float16))]

    qr, qk, qv = sb6(3 * D, D), sb6(F, D), sb6(D, F)
    rw, ra, rv, rg = syn.lora_ranks(D)
    RT = rw + ra + rv + rg
    wcat = dev((rng.standard_normal((RT, D)) * 0.05).astype(np.float16))
    f = lambda *s, scale=1.0: dev((rng.standard_normal(s) * scale).astype(np.float32))
    x, lnw, lnb, prev, coef6 = f(D, scale=2.0), f(D, scale=0.3) + 1, f(D, scale=0.1), f(D), f(6, D, scale=0.5)
    p = lambda t: t.data_ptr()
    # reference: shift_mix (6 coefficients) + rkv_lora
    prev_a, xrkv, xmix = prev.clone(), torch.empty(3, D, device=DEV), torch.empty(4, D, device=DEV)
    y_a, la_a = torch.empty(3 * D, device=DEV), torch.empty(RT, device=DEV)
    _lib.check(L.rwkv_x070_shift_mix(p(x), p(lnw), p(lnb), p(prev_a), p(coef6), 6, p(xrkv), p(xmix), 1, D, 1e-5, None))
    _lib.check(L.rwkv_x070_rkv_lora(p(xrkv), *[p(t) for t in qr], p(y_a), 3 * D, D, 0, D, p(xmix), p(wcat), _lib.F16,
                                    rw, ra, rv, rg, 1, p(la_a), None))
    y_b, la_b, xl = torch.empty(3 * D, device=DEV), torch.empty(RT, device=DEV), torch.empty(D, device=DEV)
    _lib.check(L.rwkv_x070_rkv_lora_ln(p(x), p(lnw), p(lnb), p(prev), p(coef6), 1e-5, p(xl), *[p(t) for t in qr],
                                       p(y_b), D, 0, p(wcat), _lib.F16, rw, ra, rv, rg, 1, p(la_b), None))
    torch.cuda.synchronize()
    assert torch.equal(y_a, y_b) and torch.equal(la_a, la_b)
    assert torch.equal(xl, prev_a)          # the LN row shift_mix stored as the next prev
    # ffn: shift_mix (1 coefficient) + key GEMV relu², then value + residual
    ck = coef6[1].contiguous()
    prev_c, xk, hk_a = prev.clone(), torch.empty(D, device=DEV), torch.empty(F, device=DEV)
    _lib.check(L.rwkv_x070_shift_mix(p(x), p(lnw), p(lnb), p(prev_c), p(ck), 1, p(xk), None, 1, D, 1e-5, None))
    _lib.check(L.rwkv_sb6_gemv_ep(p(xk), 1, *[p(t) for t in qk], p(hk_a), F, D, 0, 2, None))
    hk_b, xl2 = torch.empty(F, device=DEV), torch.empty(D, device=DEV)
    _lib.check(L.rwkv_x070_ffn_key_ln(p(x), p(lnw), p(lnb), p(prev), p(ck), 1e-5, p(xl2), *[p(t) for t in qk],
                                      p(hk_b), F, D, 0, None))
    torch.cuda.synchronize()
    assert torch.equal(hk_a, hk_b) and torch.equal(xl2, prev_c)
    xa, xb, dst = x.clone(), x.clone(), prev.clone()
    _lib.check(L.rwkv_sb6_gemv_ep(p(hk_a), 1, *[p(t) for t in qv], p(xa), D, F, 0, 1, None))
    _lib.check(L.rwkv_x070_ffn_value(p(hk_b), *[p(t) for t in qv], p(xb), D, F, 0, p(xl2), p(dst), None))
    torch.cuda.synchronize()
    assert torch.equal(xa, xb) and torch.equal(dst, prev_c)


@pytest.mark.parametrize("N", [1, 2])
def test_decode_graph_replay_bitwise(tiny, decoder, N):
    case(f"decode graph replay N={N}")
    st = decoder.new_state(N)
    ids = torch.tensor([3, 400][:N], dtype=torch.int32, device=DEV)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        decoder.launch(ids, st)   # one token so the state is not zero
        s0 = st.clone()
        eager = decoder.launch(ids, st).clone()
        eager_st = st.clone()
        g = torch.cuda.CUDAGraph()
        st.copy_(s0)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            out = decoder.launch(ids, st)
        torch.cuda.synchronize()
        for rep in range(3):
            st.copy_(s0)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), rep
            assert torch.equal(st.wkv, eager_st.wkv) and torch.equal(st.cmix_prev, eager_st.cmix_prev), rep


def test_generate_batch_rows_equal_prompts_alone(decoder):
    # prefillBatch / generateBatch (BatchGenerate.swift:37-116) with the
    # greedy choice: every row of the batch is bitwise its prompt alone (the
    # reference bounds it at 1e-5, BatchGenerateTests.swift:56-61; batches of
    # up to 4 rows keep the row-invariant VALU GEMVs and row kernels; 4 heads
    # keep the four-rows-per-wave WKV layout at every batch here)
    case("generate_batch tiny")
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, TINY.vocab, n).tolist() for n in (3, 5, 1)]
    logits, st = decoder.prefill_batch(prompts)
    assert logits.shape == (3, TINY.vocab)
    for i, p in enumerate(prompts):
        li, si = decoder.prefill_batch([p])
        assert torch.equal(logits[i], li[0]), i
        for a, b in ((st.wkv, si.wkv), (st.tmix_prev, si.tmix_prev), (st.cmix_prev, si.cmix_prev)):
            assert torch.equal(a[:, i], b[:, 0]), i
    out = decoder.generate_batch(prompts, 6)
    assert [len(o) for o in out] == [6, 6, 6]
    assert out == [decoder.generate_batch([p], 6)[0] for p in prompts]
    # the first token is the greedy choice of the prefill logits
    assert [o[0] for o in out] == torch.argmax(logits, dim=1).cpu().tolist()
    # a stop token ends its row (kept as the row's last token); the other
    # rows go on after it leaves the batch
    stop = out[0][2]
    out2 = decoder.generate_batch(prompts, 6, stop_tokens=[stop])
    assert out2[0] == out[0][:out[0].index(stop) + 1]
    assert out2 == [decoder.generate_batch([p], 6, stop_tokens=[stop])[0] for p in prompts]
    assert decoder.generate_batch(prompts, 0) == [[], [], []]
    with pytest.raises(ValueError):
        decoder.prefill_batch([[1, 2], []])
    with pytest.raises(ValueError):
        decoder.step_batch([1, 2], decoder.new_state(3))


@pytest.fixture(scope="module")
def proj_0b1():
    proj = syn.x070_projections(syn.X070_0B1, nthreads=8)
    return proj, X.dequant_projections(proj)


# fp32 low-rank matrices: no fp16 rounding points, so the step is fp32
# arithmetic against fp64 throughout (2e-5).  fp16 matrices (the .rwkvq norm):
# 12 layers of low-rank outputs rounded to fp16, where an fp32 sum and the
# fp64 sum may round to neighbouring fp16 values (one ulp = 2^-10 relative);
# measured 1.3e-4 on these logits, bound 5e-4.
@pytest.mark.parametrize("lora", ["f32", "f16"])
def test_decode_0b1_shape_matches_oracle(proj_0b1, lora):
    case(f"decode 0.1B shape, low-rank {lora}, 2 tokens")
    shape = syn.X070_0B1
    p = syn.x070_dense_params(shape, seed=5, lora_dtype=np.float32 if lora == "f32" else np.float16)
    proj, W = proj_0b1
    d = X070Decoder(shape.n_layer, shape.n_embd, shape.ffn, shape.vocab, p, proj, DEV)
    st = d.new_state(1)
    ost = X.State.zeros(shape.n_layer, 1, shape.n_head)
    tol = 2e-5 if lora == "f32" else 5e-4
    for t, i in enumerate((11, 40000)):
        got = d.step([i], st).cpu().numpy()
        ref = X.step(p, W, [i], ost, shape.n_layer, shape.n_head)
        err = rel(ref, got)
        print(f"[x070] 0.1B low-rank {lora} token {t}: rel {err:.3e}", flush=True)
        assert err < tol, t


def test_decoder_from_rwkvq_file(tmp_path, orc):
    """A full .rwkvq export (world naming, dense body) with mixed projection
    kinds: layer 0 r/k/v sb6 (one fused sb6 GEMV), o_proj dense (as current
    presets store it), layer 1 r/k/v sym 8-bit (one fused sym GEMV), sym
    ffn, sym head; decoded through X070Decoder.from_sidecar against the oracle
    on the matrices dequantised from the disk buffers."""
    from swiftrwkv_amd import quant as Q
    from tests.test_x070_oracle import file_projections, world_file
    case("decoder from .rwkvq file, mixed kinds")
    p = syn.x070_dense_params(TINY, seed=9)
    kinds = {"blocks.0.att.output.weight": "dense", "head.weight": "sym8"}
    kinds.update({f"blocks.1.att.{m}.weight": "sym8" for m in ("receptance", "key", "value")})
    kinds.update({f"blocks.1.ffn.{m}.weight": "sym8" for m in ("key", "value")})
    path = str(tmp_path / "tiny.rwkvq")
    T = world_file(path, TINY, p, kinds)
    sc = Q.RwkvqSidecar.from_rwkvq(path)
    dec = X070Decoder.from_sidecar(sc)
    from swiftrwkv_amd.x070 import Proj
    assert isinstance(dec.proj["blocks.0.att.rkv"], Proj) and dec.proj["blocks.0.att.rkv"].kind == "sb6"
    assert isinstance(dec.proj["blocks.1.att.rkv"], Proj) and dec.proj["blocks.1.att.rkv"].kind == "sym"
    assert dec.proj["blocks.0.att.output.weight"].kind == "dense"
    W = file_projections(orc, T, TINY)
    for N in (1, 2):
        st = dec.new_state(N)
        ost = X.State.zeros(TINY.n_layer, N, TINY.n_head)
        rng = np.random.default_rng(N)
        for t in range(3):
            ids = rng.integers(0, TINY.vocab, N).astype(np.int32)
            got = dec.step(ids, st).cpu().numpy()
            ref = X.step(p, W, ids, ost, TINY.n_layer, TINY.n_head)
            assert rel(ref, got) < 1e-4, (N, t)
