"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Every oracle function is checked against something that does not share its
code: numpy / torch IEEE conversions, an independent bit-stream reader, numpy
packers and formulas written from the *generated* codes rather than from the
packed bytes, matrix-form (numpy matmul) restatements of the recurrence,
closed forms (T = 1, gated / causal linear attention), central finite
differences, the reference's in-repo known-answer test, and the reference's
own bitwise invariants (split == contiguous, neutral pad step).
"""
import json
import os

import numpy as np
import pytest
import torch

from swiftrwkv_amd import synthetic as syn

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ───────────────────────────── conversions ─────────────────────────────

def test_f32_to_f16_matches_numpy(orc):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200_000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 200_000),
        np.float32([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 1e-10]),
    ]).astype(np.float32)
    # exact ties between neighbouring halves (normal and subnormal range)
    h = rng.integers(0, 0x7bff, 50_000).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float32)
    hi = (h + 1).view(np.float16).astype(np.float32)
    ties = ((lo.astype(np.float64) + hi.astype(np.float64)) / 2).astype(np.float32)
    x = np.concatenate([x, ties, -ties])
    want = x.astype(np.float16).view(np.uint16)
    got = orc.f32_to_f16_bits(x)
    assert np.array_equal(got, want)


def test_f16_to_f32_all_patterns(orc):
    h = np.arange(65536, dtype=np.uint16)
    finite = (h & 0x7c00) != 0x7c00
    want = h.view(np.float16).astype(np.float32)
    got = orc.f16_bits_to_f32(h)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isinf(got[(h & 0x7fff) == 0x7c00]))


def test_f32_to_bf16_matches_torch(orc):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(300_000) * 10.0 ** rng.integers(-20, 20, 300_000)).astype(np.float32)
    base = rng.integers(0, 0x7f00, 20_000).astype(np.uint32) << 16
    ties = (base | 0x8000).view(np.float32)                 # exactly halfway
    x = np.concatenate([x, ties, -ties, np.float32([0.0, -0.0, 3.4e38])])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.f32_to_bf16_bits(x), want)


# ───────────────────────────── unpack6 / K3 / sym interleave ─────────────────────────────

def _bitstream_unpack6(b):
    """Independent reader: LSB-first bit stream, 6 bits per value."""
    bits = np.unpackbits(b.reshape(-1, 6), axis=1, bitorder="little").reshape(-1, 8, 6)
    return (bits.astype(np.int32) * (1 << np.arange(6, dtype=np.int32))).sum(-1)


def test_unpack6x8_exhaustive_over_three_byte_chunks(orc):
    # every 3-byte chunk in the first half of a group, a varying chunk in the second
    rng = np.random.default_rng(2)
    for start in range(0, 1 << 24, 1 << 20):
        v = np.arange(start, start + (1 << 20), dtype=np.uint32)
        g = np.empty((1 << 20, 6), np.uint8)
        g[:, 0], g[:, 1], g[:, 2] = v & 0xff, (v >> 8) & 0xff, v >> 16
        g[:, 3:] = rng.integers(0, 256, (1 << 20, 3), dtype=np.uint8)
        assert np.array_equal(orc.unpack6x8(g), _bitstream_unpack6(g))


def _pack6(vals):
    """Independent writer: values [..., 8] (0..63) → bytes [..., 6], LSB-first."""
    v = np.asarray(vals, np.uint8)
    bits = np.unpackbits(v[..., None], axis=-1, bitorder="little")[..., :6]
    return np.packbits(bits.reshape(v.shape[:-1] + (48,)), axis=-1, bitorder="little")


def make_sb6(OUT, IN, xbits, rng, degenerate=False):
    """Random sb6 tensor: the generated codes/scales and their DISK layout."""
    NB, NSB = IN // 32, IN // 256
    codes = rng.integers(0, 1 << (4 + xbits), (OUT, NB, 32))
    qs = rng.integers(0, 64, (OUT, NB))
    qm = rng.integers(-31, 33, (OUT, NB))
    if degenerate:
        qs[:, ::5] = 0
    d = (rng.uniform(1e-4, 3e-3, (OUT, NSB))).astype(np.float16)
    dm = (rng.uniform(1e-4, 3e-3, (OUT, NSB))).astype(np.float16)
    cp = ((codes[:, :, :16] & 0xf) | ((codes[:, :, 16:] & 0xf) << 4)).astype(np.uint8).reshape(OUT, NB * 16)
    planes = []
    for bit in range(4, 4 + xbits):
        bitsv = ((codes >> bit) & 1).astype(np.uint8)
        planes.append(np.packbits(bitsv, axis=-1, bitorder="little").reshape(OUT, NB * 4))
    qh = planes[0] if xbits >= 1 else None
    qh2 = planes[1] if xbits >= 2 else None
    qsqm_disk = np.concatenate([_pack6(qs.reshape(OUT, NSB, 8)), _pack6((qm + 31).reshape(OUT, NSB, 8))], -1)
    return dict(codes=codes, qs=qs, qm=qm, d=d, dm=dm, cp=cp, qh=qh, qh2=qh2, qsqm_disk=qsqm_disk)


def sb6_expected(t):
    """Dequant written from the generated codes (numpy float16 as `half`)."""
    OUT, NB = t["qs"].shape
    d = np.repeat(t["d"].astype(np.float32), 8, axis=1)
    dm = np.repeat(t["dm"].astype(np.float32), 8, axis=1)
    s = (t["qs"].astype(np.float32) * d).astype(np.float16).astype(np.float32)
    m = (t["qm"].astype(np.float32) * dm).astype(np.float16).astype(np.float32)
    w = t["codes"].astype(np.float32) * s[..., None] + m[..., None]
    return w.reshape(OUT, NB * 32).astype(np.float32)


@pytest.mark.parametrize("xbits", [0, 1, 2])
def test_sb6_k3_and_dequant_against_generated_codes(orc, xbits):
    rng = np.random.default_rng(10 + xbits)
    OUT, IN = 12, 768
    t = make_sb6(OUT, IN, xbits, rng, degenerate=True)
    qblk, qsqm, ddm, xb = orc.sb6_to_k3(t["cp"], t["qh"], t["qh2"], t["qsqm_disk"], t["d"].view(np.uint16),
                                        t["dm"].view(np.uint16), OUT, IN)
    assert xb == xbits
    NB = IN // 32
    SU = 16 + 4 * xbits
    blk = qblk.reshape(OUT, NB, SU)
    assert np.array_equal(blk[:, :, :16].reshape(OUT, -1), t["cp"])
    if xbits:
        assert np.array_equal(blk[:, :, 16:20].reshape(OUT, -1), t["qh"])
    k3 = qsqm.reshape(OUT, NB, 2)
    assert np.array_equal(k3[:, :, 0], t["qs"])
    assert np.array_equal(k3[:, :, 1].view(np.int8), t["qm"].astype(np.int8))
    w = orc.sb6_dequant(qblk, qsqm, ddm, OUT, IN, xbits)
    want = sb6_expected(t)
    assert np.array_equal(w.view(np.uint32), want.view(np.uint32))
    # degenerate blocks (qs = 0 ⇒ s = 0) give w = m exactly (RwkvqSb6GEMV.swift:29-33)
    dg = (t["qs"] == 0)
    m = (t["qm"].astype(np.float32) * np.repeat(t["dm"].astype(np.float32), 8, 1)).astype(np.float16).astype(np.float32)
    assert np.array_equal(w.reshape(OUT, NB, 32)[dg], np.broadcast_to(m[dg][:, None], (dg.sum(), 32)))
    # bf16 / f16 storage = one rounding of the fp32 value (RwkvqDTypeTests.swift:39-58)
    wb = orc.sb6_dequant(qblk, qsqm, ddm, OUT, IN, xbits, "bf16")
    assert np.array_equal(wb, torch.from_numpy(want).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    wh = orc.sb6_dequant(qblk, qsqm, ddm, OUT, IN, xbits, "f16")
    assert np.array_equal(wh, want.astype(np.float16).view(np.uint16))


def make_sym(OUT, IN, bits, rng):
    NB = IN // 16
    NSB = (NB + 15) // 16
    lo, hi = (-128, 128) if bits == 8 else (-32, 32)
    q = rng.integers(lo, hi, (OUT, IN))
    qs = rng.integers(-128, 128, (OUT, NB)).astype(np.int8)
    d = rng.uniform(1e-4, 2e-3, (OUT, NSB)).astype(np.float16)
    t = dict(q=q, qs=qs, d=d)
    if bits == 8:
        t["qblk"] = q.astype(np.int8).view(np.uint8)
    else:
        st = (q + 32).reshape(OUT, IN // 32, 2, 16)   # pair, block, column
        cp = ((st[..., :8] & 0xf) | ((st[..., 8:] & 0xf) << 4)).astype(np.uint8).reshape(OUT, IN // 32 * 16)
        planes = [np.packbits(((q + 32).reshape(OUT, IN // 32, 32) >> bit & 1).astype(np.uint8), axis=-1,
                              bitorder="little").reshape(OUT, IN // 32 * 4) for bit in (4, 5)]
        t.update(cp=cp, qh=planes[0], qh2=planes[1])
    return t


def sym_expected(t):
    OUT, IN = t["q"].shape
    NB = IN // 16
    dd = np.repeat(t["d"].astype(np.float32), 16, axis=1)[:, :NB]
    s = (t["qs"].astype(np.float32) * dd).astype(np.float16).astype(np.float32)
    return (t["q"].reshape(OUT, NB, 16).astype(np.float32) * s[..., None]).reshape(OUT, IN)


@pytest.mark.parametrize("bits", [8, 6])
def test_sym_interleave_and_dequant_against_generated_codes(orc, bits):
    rng = np.random.default_rng(20 + bits)
    OUT, IN = 10, 512
    t = make_sym(OUT, IN, bits, rng)
    qblk = t["qblk"] if bits == 8 else orc.sym_interleave(t["cp"], t["qh"], t["qh2"], OUT, IN)
    if bits == 6:
        pr = qblk.reshape(OUT, IN // 32, 24)
        assert np.array_equal(pr[:, :, :16].reshape(OUT, -1), t["cp"])
        assert np.array_equal(pr[:, :, 20:].reshape(OUT, -1), t["qh2"])
    w = orc.sym_dequant(qblk, t["qs"].view(np.uint8), t["d"].view(np.uint16), OUT, IN, bits)
    want = sym_expected(t)
    assert np.array_equal(w.view(np.uint32), want.view(np.uint32))
    wh = orc.sym_dequant(qblk, t["qs"].view(np.uint8), t["d"].view(np.uint16), OUT, IN, bits, "f16")
    assert np.array_equal(wh, want.astype(np.float16).view(np.uint16))


def test_sym8_known_answer_from_reference_test(orc):
    kat = json.load(open(os.path.join(GOLD, "sym8_kat.json")))
    OUT, IN = kat["OUT"], kat["IN"]
    w = orc.sym_dequant(np.array(kat["codes_u8"], np.uint8), np.array(kat["qs_u8"], np.uint8),
                        np.array(kat["d_f16_bits"], np.uint16), OUT, IN, 8)
    assert np.array_equal(w.reshape(-1), np.array(kat["expected_f32"], np.float32))


# ───────────────────────────── GEMV anchors ─────────────────────────────

def test_gemv_one_hot_gives_dequant_columns(orc):
    rng = np.random.default_rng(30)
    OUT, IN = 16, 512
    t = make_sb6(OUT, IN, 1, rng)
    qblk, qsqm, ddm, xb = orc.sb6_to_k3(t["cp"], t["qh"], t["qh2"], t["qsqm_disk"], t["d"].view(np.uint16),
                                        t["dm"].view(np.uint16), OUT, IN)
    W = orc.sb6_dequant(qblk, qsqm, ddm, OUT, IN, xb)
    cols = [0, 17, 255, 256, 511]
    x = np.zeros((len(cols), IN), np.float32)
    x[np.arange(len(cols)), cols] = 1.0
    y = orc.sb6_gemv_f64(x, qblk, qsqm, ddm, OUT, IN, xb)
    assert np.array_equal(y, W[:, cols].T.astype(np.float64))
    xr = rng.standard_normal((3, IN)).astype(np.float32)
    assert np.allclose(orc.sb6_gemv_f64(xr, qblk, qsqm, ddm, OUT, IN, xb),
                       xr.astype(np.float64) @ W.T.astype(np.float64), rtol=1e-12, atol=1e-12)
    s = make_sym(OUT, IN, 6, rng)
    sq = orc.sym_interleave(s["cp"], s["qh"], s["qh2"], OUT, IN)
    Ws = orc.sym_dequant(sq, s["qs"].view(np.uint8), s["d"].view(np.uint16), OUT, IN, 6)
    ys = orc.sym_gemv_f64(x, sq, s["qs"].view(np.uint8), s["d"].view(np.uint16), OUT, IN, 6)
    assert np.array_equal(ys, Ws[:, cols].T.astype(np.float64))
    # fused: K = 2 matrices of 8 rows, row o of input n reads x[n·2 + o // 8]
    xf = rng.standard_normal((2, IN)).astype(np.float32)
    yf = orc.sym_gemv_f64(xf, sq, s["qs"].view(np.uint8), s["d"].view(np.uint16), OUT, IN, 6, out_per=8)
    want = np.concatenate([Ws[:8].astype(np.float64) @ xf[0].astype(np.float64),
                           Ws[8:].astype(np.float64) @ xf[1].astype(np.float64)])
    assert np.allclose(yf[0], want, rtol=1e-12, atol=1e-12)


# ───────────────────────────── WKV-7 forward ─────────────────────────────

def _matrix_form_f64(r, w, k, v, a, b, h0=None):
    """S_t = S_{t-1}(diag(w_t) + a_t b_tᵀ) + v_t k_tᵀ ; y_t = S_t r_t (numpy matmuls)."""
    B, T, H, D = r.shape
    r, w, k, v, a, b = (x.astype(np.float64) for x in (r, w, k, v, a, b))
    S = np.zeros((B, H, D, D)) if h0 is None else h0.astype(np.float64).copy()
    out = np.empty((B, T, H, D))
    for t in range(T):
        G = np.einsum("bhj,bhjk->bhjk", w[:, t], np.broadcast_to(np.eye(D), (B, H, D, D))) \
            + a[:, t, :, :, None] * b[:, t, :, None, :]
        S = S @ G + v[:, t, :, :, None] * k[:, t, :, None, :]
        out[:, t] = (S @ r[:, t, :, :, None])[..., 0]
    return out, S


def test_fwd_matches_matrix_form_and_fp32_order(orc):
    x = syn.wkv_inputs_train(2, 24, 3, seed=5)
    h0 = syn.state(2, 3, seed=6)
    o64, s64 = orc.wkv7_fwd_f64(*x, h_in=h0)
    om, sm = _matrix_form_f64(*x, h0=h0)
    assert np.allclose(o64, om, rtol=1e-11, atol=1e-11) and np.allclose(s64, sm, rtol=1e-11, atol=1e-11)
    o32, s32 = orc.wkv7_fwd_f32(*x, h_in=h0)
    rel = np.abs(o32 - o64).max() / np.abs(o64).max()
    assert rel < 1e-5


def test_fwd_closed_forms(orc):
    rng = np.random.default_rng(3)
    B, H, D = 1, 2, 64
    # (1) zero state, one token: S = v kᵀ, y = v (k·r)
    x = syn.wkv_inputs_train(B, 1, H, seed=1)
    o, s = orc.wkv7_fwd_f64(*x)
    r, w, k, v, a, b = (z.astype(np.float64) for z in x)
    assert np.allclose(s[0], v[0, 0, :, :, None] * k[0, 0, :, None, :], rtol=0, atol=1e-15)
    assert np.allclose(o[0, 0], v[0, 0] * (k[0, 0] * r[0, 0]).sum(-1, keepdims=True), rtol=1e-13, atol=1e-15)
    # (2) a = b = 0: gated linear attention with an initial state
    T = 9
    x = syn.wkv_inputs_train(B, T, H, seed=2)
    x[4][:] = 0
    x[5][:] = 0
    h0 = syn.state(B, H, seed=4)
    o, _ = orc.wkv7_fwd_f64(*x, h_in=h0)
    r, w, k, v = (z.astype(np.float64)[0] for z in x[:4])
    want = np.zeros((T, H, D))
    for t in range(T):
        decay0 = np.prod(w[:t + 1], axis=0)                               # [H, D] over j
        want[t] += np.einsum("hij,hj,hj->hi", h0[0].astype(np.float64), decay0, r[t])
        for s_ in range(t + 1):
            dec = np.prod(w[s_ + 1:t + 1], axis=0) if s_ < t else np.ones((H, D))
            want[t] += v[s_] * (k[s_] * r[t] * dec).sum(-1)[:, None]
    assert np.allclose(o[0], want, rtol=1e-12, atol=1e-12)
    # (3) additionally w = 1: causal linear attention (R Kᵀ ⊙ causal) V
    x[1][:] = 1.0
    o, _ = orc.wkv7_fwd_f64(*x)
    r, _, k, v = (z.astype(np.float64)[0] for z in x[:4])
    for hh in range(H):
        A = np.tril(r[:, hh] @ k[:, hh].T)
        assert np.allclose(o[0, :, hh], A @ v[:, hh], rtol=1e-12, atol=1e-12)


def test_fwd_split_contiguous_and_pad_bitwise(orc):
    x = syn.wkv_inputs_seq(1, 41, 3, seed=7)
    o, h = orc.wkv7_fwd_f32(*x)
    o1, h1 = orc.wkv7_fwd_f32(*[z[:, :19] for z in x])
    o2, h2 = orc.wkv7_fwd_f32(*[z[:, 19:] for z in x], h_in=h1)
    assert np.array_equal(np.concatenate([o1, o2], 1), o) and np.array_equal(h2, h)
    # neutral steps (w = 1, others 0) leave the state unchanged
    pad = [np.zeros((1, 5, 3, 64), np.float32) for _ in range(6)]
    pad[1][:] = 1.0
    _, hp = orc.wkv7_fwd_f32(*[np.concatenate([z, p], 1) for z, p in zip(x, pad)])
    assert np.array_equal(hp, h)


def test_fwd_checkpoints_and_sa(orc):
    x = syn.wkv_inputs_train(1, 32, 2, seed=8)
    o, h, sa, ck = orc.wkv7_fwd_f32(*x, want_sa=True, want_ckpt=True)
    _, h16 = orc.wkv7_fwd_f32(*[z[:, :16] for z in x])
    assert np.array_equal(ck[:, :, 0], h16) and np.array_equal(ck[:, :, 1], h)
    _, _, sa64 = orc.wkv7_fwd_f64(*x, want_sa=True)
    assert np.abs(sa - sa64).max() / np.abs(sa64).max() < 1e-5


# ───────────────────────────── WKV-7 backward ─────────────────────────────

def test_bwd_matches_central_finite_differences(orc):
    B, T, H = 1, 6, 1
    rng = np.random.default_rng(9)
    x = [z.astype(np.float64) for z in syn.wkv_inputs_train(B, T, H, seed=9)]
    h0 = syn.state(B, H, seed=10).astype(np.float64)
    g = rng.standard_normal((B, T, H, 64))
    gh = rng.standard_normal((B, H, 64, 64)) * 0.3

    def loss(xs, h):
        o, s = orc.wkv7_fwd_f64(*xs, h_in=h)
        return (o * g).sum() + (s * gh).sum()

    grads = orc.wkv7_bwd_f64(*x, h0, g, gh)
    eps = 1e-6
    for which in range(6):
        for _ in range(12):
            idx = tuple(rng.integers(0, n) for n in x[which].shape)
            xp = [z.copy() for z in x]
            xm = [z.copy() for z in x]
            xp[which][idx] += eps
            xm[which][idx] -= eps
            fd = (loss(xp, h0) - loss(xm, h0)) / (2 * eps)
            assert abs(fd - grads[which][idx]) <= 1e-6 * max(1.0, abs(fd)), (which, idx, fd, grads[which][idx])
    for _ in range(12):
        idx = tuple(rng.integers(0, n) for n in h0.shape)
        hp, hm = h0.copy(), h0.copy()
        hp[idx] += eps
        hm[idx] -= eps
        fd = (loss(x, hp) - loss(x, hm)) / (2 * eps)
        assert abs(fd - grads[6][idx]) <= 1e-6 * max(1.0, abs(fd))


def test_bwd_dr_through_final_state_only_is_exactly_zero(orc):
    # WKV7StateTests.swift:240-262: y reads the updated state, the update does not read r.
    x = syn.wkv_inputs_train(1, 16, 2, seed=11)
    gh = syn.state(1, 2, scale=0.3, seed=12)
    grads = orc.wkv7_bwd_f64(*x, None, np.zeros((1, 16, 2, 64)), gh)
    assert np.abs(grads[0]).max() == 0.0
    assert np.abs(grads[2]).max() > 0.0


# ───────────────────────────── tail ─────────────────────────────

def test_tail_formula_and_closed_form(orc):
    rng = np.random.default_rng(13)
    for H in (12, 32):
        S, N = 64, 3
        D = H * S
        wkv = (rng.standard_normal((N, H, S)) * 3).astype(np.float32)
        r, k, v = (rng.standard_normal((N, H, S)).astype(np.float32) for _ in range(3))
        rk = (rng.standard_normal((H, S)) * 0.1).astype(np.float32)
        lnw = (rng.standard_normal(D) * 0.5 + 1).astype(np.float32)
        lnb = (rng.standard_normal(D) * 0.1).astype(np.float32)
        g = rng.standard_normal((N, D)).astype(np.float32)
        got = orc.wkv_tail_f64(wkv, r, k, v, rk, lnw, lnb, g, N, H, S)
        x = wkv.astype(np.float64)
        mean = x.mean(-1, keepdims=True)
        var = ((x - mean) ** 2).mean(-1, keepdims=True)
        normed = ((x - mean) / np.sqrt(var + 64e-5)).reshape(N, D) * lnw + lnb
        bonus = ((r.astype(np.float64) * k * rk).sum(-1, keepdims=True) * v).reshape(N, D)
        assert np.allclose(got, (normed + bonus) * g, rtol=1e-12, atol=1e-12)
        # constant wkv per head: the normalised part vanishes exactly
        c = np.broadcast_to(rng.standard_normal((N, H, 1)).astype(np.float32), (N, H, S)).copy()
        got = orc.wkv_tail_f64(c, r, k, v, rk, lnw, lnb, g, N, H, S)
        want = (lnb + ((r.astype(np.float64) * k * rk).sum(-1, keepdims=True) * v).reshape(N, D)) * g
        assert np.allclose(got, want, rtol=1e-13, atol=1e-13)


@pytest.mark.parametrize("xbits", [0, 1])
def test_cpu_baseline_matvec_matches_fp64(orc, xbits):
    """The timed CPU restatement of the non-kernel projection path (dequantise
    to fp32, fp32 x·Wᵀ) agrees with the fp64 anchor, on any thread count."""
    OUT, IN = 96, 1024
    t = make_sb6(OUT, IN, xbits, np.random.default_rng(30 + xbits))
    qblk, qsqm, ddm, xb = orc.sb6_to_k3(t["cp"], t["qh"], t["qh2"], t["qsqm_disk"], t["d"].view(np.uint16),
                                        t["dm"].view(np.uint16), OUT, IN)
    x = np.random.default_rng(31).standard_normal(IN).astype(np.float32)
    want = orc.sb6_gemv_f64(x[None], qblk, qsqm, ddm, OUT, IN, xb)[0]
    y1 = orc.cpu_sb6_dequant_matvec(x, qblk, qsqm, ddm, OUT, IN, xb, 1)
    y4 = orc.cpu_sb6_dequant_matvec(x, qblk, qsqm, ddm, OUT, IN, xb, 4)
    assert np.array_equal(y1, y4)
    assert np.abs(y1 - want).max() / np.abs(want).max() < 2e-5


def test_cpu_baseline_wkv_step_matches_fp64(orc):
    """The timed CPU decode step (B rows, in place) against the fp64 forward
    at T = 1 from the same state."""
    from swiftrwkv_amd import synthetic as syn
    B, H = 2, 3
    x = syn.wkv_inputs_config0(B, 1, H, seed=32)
    h0 = syn.state(B, H, scale=0.5, seed=33)
    o64, h64 = orc.wkv7_fwd_f64(*x, h0)
    vec = [np.ascontiguousarray(z[:, 0]) for z in x]
    outs = []
    for nt in (1, 4):
        h = h0.copy()
        out = np.empty((B, H, 64), np.float32)
        orc.cpu_wkv7_step(*vec, h, out, B, H, nt)
        outs.append((out, h))
        assert np.abs(out - o64[:, 0]).max() / np.abs(o64).max() < 1e-5
        assert np.abs(h - h64).max() / np.abs(h64).max() < 1e-5
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])


def test_f16_base_matmul_oracle(orc):
    """The fp16-base long-pass anchor: one-hot inputs give the fp16 dequant
    column exactly (a value exact in fp16 passes unrounded); an input that is
    not an fp16 value is rounded (RNE) before the product; the magnitude is
    Σ|x·w|."""
    OUT, IN = 64, 512
    t = make_sb6(OUT, IN, 0, np.random.default_rng(40))
    qblk, qsqm, ddm, _ = orc.sb6_to_k3(t["cp"], None, None, t["qsqm_disk"], t["d"].view(np.uint16),
                                       t["dm"].view(np.uint16), OUT, IN)
    w16 = sb6_expected(t).astype(np.float16).astype(np.float64)   # one rounding of the fp32 dequant
    for j in (0, 77, 511):
        x = np.zeros((1, IN), np.float32)
        x[0, j] = 1.0
        exact, mag = orc.sb6_matmul_f16_base(x, qblk, qsqm, ddm, OUT, IN)
        assert np.array_equal(exact[0], w16[:, j]) and np.array_equal(mag[0], np.abs(w16[:, j]))
    x = np.zeros((1, IN), np.float32)
    x[0, 5] = np.float32(1.0 + 2.0 ** -12)        # between fp16 neighbours 1 and 1 + 2^-10: rounds to 1
    x[0, 9] = np.float32(1.0 + 3 * 2.0 ** -11)    # a tie: rounds to even, 1 + 2^-9
    exact, _ = orc.sb6_matmul_f16_base(x, qblk, qsqm, ddm, OUT, IN)
    assert np.allclose(exact[0], w16[:, 5] + (1.0 + 2.0 ** -9) * w16[:, 9], rtol=0, atol=1e-15)
