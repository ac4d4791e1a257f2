"""Pins of the x070 decode-step oracle (oracle/x070.py), CPU only.

* layer_norm / l2norm against torch's own layer_norm / normalize (fp64);
* the fp16 rounding points (`lin`, X070Generation.swift:248-253): round to
  nearest even, input and product rounded, fp32 matrices untouched;
* the per-token step against the whole-sequence formulation (token shift as a
  shifted copy, the WKV over all steps at once): the reference's own check
  that the parallel prefill and the recurrent one agree
  (X070Generation.swift:369-376);
* v_first does not cross a step (X070Generation.swift:50-57: zeroing it
  before `step` leaves the logits unchanged);
* rows of a batch are independent;
* the decay constant, by RWKV-7's log-decay form (the step and the sequence
  share `decay`, so their agreement cannot catch a wrong constant).
"""
import numpy as np
import pytest
import torch

from oracle import x070 as X
from swiftrwkv_amd import synthetic as syn

TINY = syn.X070Shape("tiny", 2, 256, 1024, vocab=512)


def test_decay_matches_log_decay_form():
    """RWKV-7 forms the log decay as w = −softplus(−z) − 1/2 and decays by
    exp(−exp(w)); exp(−softplus(−z)) = σ(z), so the decay is exp(−e^{−1/2}·σ(z)),
    and the reference's 0.606531 is e^{−1/2} to six figures.  A wrong constant,
    a missing sigmoid or a sign slip fails at this tolerance."""
    z = np.linspace(-30.0, 30.0, 2001)
    want = np.exp(-np.exp(-np.logaddexp(0.0, -z) - 0.5))
    np.testing.assert_allclose(X.decay(z), want, rtol=2e-6, atol=0.0)


@pytest.fixture(scope="module")
def tiny():
    p = syn.x070_dense_params(TINY, seed=3)
    W = X.dequant_projections(syn.x070_projections(TINY, nthreads=4))
    return p, W


def test_layer_norm_matches_torch():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 768)) * 3 + 1
    w, b = rng.standard_normal(768), rng.standard_normal(768)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x), (768,), torch.from_numpy(w), torch.from_numpy(b),
                                         eps=1e-5).numpy()
    np.testing.assert_allclose(X.layer_norm(x, w, b), ref, rtol=0, atol=1e-12)


def test_l2norm_heads_matches_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 4 * 64))
    ref = torch.nn.functional.normalize(torch.from_numpy(x).reshape(3, 4, 64), dim=-1).reshape(3, 256).numpy()
    np.testing.assert_allclose(X.l2norm_heads(x, 4), ref, rtol=0, atol=1e-12)


def test_f16_rounding_points():
    u = 2.0 ** -10   # fp16 ulp at 1
    # ties go to even; values between round to the nearer neighbour
    np.testing.assert_array_equal(X.f16r([1 + u / 2, 1 + 3 * u / 2, 1 + 0.51 * u, 65504.0]),
                                  [1.0, 1 + 2 * u, 1 + u, 65504.0])
    rng = np.random.default_rng(2)
    y = rng.standard_normal((2, 64))
    m16 = rng.standard_normal((32, 64)).astype(np.float16)
    out = X.lin(y, m16)
    np.testing.assert_array_equal(out, X.f16r(out))            # product rounded to fp16
    np.testing.assert_array_equal(out, X.lin(X.f16r(y), m16))   # input rounded to fp16
    m32 = m16.astype(np.float32)
    np.testing.assert_allclose(X.lin(y, m32), y @ m32.astype(np.float64).T, rtol=0, atol=1e-12)
    # exactly representable operands: the rounding points change nothing
    yi = np.array([[1.0, -2.0, 0.5, 0.0]])
    mi = np.array([[2.0, 1.0, 4.0, 7.0], [0.25, 0.5, -1.0, 3.0]], np.float16)
    np.testing.assert_array_equal(X.lin(yi, mi), [[2.0, -1.25]])


def test_step_matches_sequence(tiny):
    p, W = tiny
    ids = [5, 17, 300, 17, 2, 511]
    seq = X.sequence(p, W, ids, TINY.n_layer, TINY.n_head)
    st = X.State.zeros(TINY.n_layer, 1, TINY.n_head)
    for t, i in enumerate(ids):
        lg = X.step(p, W, [i], st, TINY.n_layer, TINY.n_head)
        np.testing.assert_allclose(lg[0], seq[t], rtol=0, atol=1e-9 * np.abs(seq[t]).max())


def test_v_first_does_not_cross_steps(tiny):
    p, W = tiny
    st = X.State.zeros(TINY.n_layer, 1, TINY.n_head)
    X.step(p, W, [7], st, TINY.n_layer, TINY.n_head)
    a, b = st.copy(), st.copy()
    b.v_first[:] = 0.0
    la = X.step(p, W, [9], a, TINY.n_layer, TINY.n_head)
    lb = X.step(p, W, [9], b, TINY.n_layer, TINY.n_head)
    np.testing.assert_array_equal(la, lb)


def test_rows_are_independent(tiny):
    p, W = tiny
    st2 = X.State.zeros(TINY.n_layer, 2, TINY.n_head)
    two = [X.step(p, W, ids, st2, TINY.n_layer, TINY.n_head) for ids in ([1, 2], [3, 4])]
    for row in range(2):
        st1 = X.State.zeros(TINY.n_layer, 1, TINY.n_head)
        for t, ids in enumerate(([1, 2], [3, 4])):
            one = X.step(p, W, [ids[row]], st1, TINY.n_layer, TINY.n_head)
            np.testing.assert_allclose(one[0], two[t][row], rtol=0, atol=1e-12 * np.abs(one).max())


# ───────────── a full .rwkvq export (world naming) and its dense body ─────────────

def world_file(path, shape, p, kinds, nthreads=4):
    """Write x070 parameters `p` (x070 names, flat vectors) as a full .rwkvq
    export in world naming: dense body as the reference's converter reads it
    (token-shift and k_k / k_a / r_k vectors [1, 1, D], w0 / a0 / v0 [1, 1, D],
    low-rank matrices raw [in, out] with `transposed` on layer 0 and Linear
    [out, in] on the others), projections encoded per `kinds` (world key →
    "sb6" / "sym8" / "dense"), the embedding dense fp16."""
    from swiftrwkv_amd import quant as Q
    D = shape.n_embd
    T = {}
    dense = lambda a, **m: ({"kind": "dense", "shape": list(np.shape(a)), **m},
                            {"dense": np.ascontiguousarray(a, np.float16)})
    vec = lambda a: dense(np.asarray(a).reshape(1, 1, D))
    T["blocks.0.ln0.weight"], T["blocks.0.ln0.bias"] = dense(p["ln0.weight"]), dense(p["ln0.bias"])
    T["ln_out.weight"], T["ln_out.bias"] = dense(p["ln_out.weight"]), dense(p["ln_out.bias"])
    T["emb.weight"] = dense(p["emb.weight"])
    for l in range(shape.n_layer):
        b, t = f"blocks.{l}.", f"blocks.{l}.tmix."
        att = b + "att."
        for n in ("ln1", "ln2"):
            T[b + n + ".weight"], T[b + n + ".bias"] = dense(p[b + n + ".weight"]), dense(p[b + n + ".bias"])
        for c in "rwkvag":
            T[att + "x_" + c] = vec(p[t + "x_" + c])
        for c in ("k_k", "k_a", "r_k"):
            T[att + c] = vec(p[t + c])
        for nm in "wavg":
            A, B = p[t + nm + "_lora_A.weight"], p[t + nm + "_lora_B.weight"]
            if l == 0:   # raw world orientation, [in, out]
                T[att + nm + "1"] = dense(A.T, transposed=True)
                T[att + nm + "2"] = dense(B.T, transposed=True)
            else:
                T[att + nm + "1"] = dense(A, transposed=False)
                T[att + nm + "2"] = dense(B, transposed=False)
            if nm != "g":
                T[att + nm + "0"] = vec(p[t + nm + "_lora_B.bias"])
        T[att + "ln_x.weight"], T[att + "ln_x.bias"] = dense(p[t + "ln_x.weight"]), dense(p[t + "ln_x.bias"])
        T[b + "ffn.x_k"] = vec(p[b + "cmix.x_k"])
    for idx, (key, OUT, IN) in enumerate(shape.projections()):
        w = (np.random.default_rng(500 + idx).standard_normal((OUT, IN)) * 0.02).astype(np.float32)
        k = kinds.get(key, "sb6")
        if k == "sb6":
            T[key] = Q.sb6_entry(w, 4, nthreads)
        elif k == "sym8":
            T[key] = Q.sym_entry(w, 8, nthreads)
        else:
            T[key] = dense(w)
    Q.write_rwkvq(path, T, n_layer=shape.n_layer, n_embd=D, vocab_size=shape.vocab)
    return T


def test_build_dense_weights_round_trip(tmp_path):
    from swiftrwkv_amd import quant as Q
    p = syn.x070_dense_params(TINY, seed=9)
    path = str(tmp_path / "tiny.rwkvq")
    world_file(path, TINY, p, {})
    sc = Q.RwkvqSidecar.from_rwkvq(path, device="cpu")
    got = sc.build_dense_weights(torch.float16)
    H = TINY.n_head
    for k, v in p.items():
        if ".v_lora_" in k and k.startswith("blocks.0."):
            assert k not in got, k   # layer 0 has no value-residual branch
            continue
        g = got[k].numpy()
        want = np.asarray(v).astype(np.float16)
        if k.endswith(("k_k", "k_a", "r_k")):
            want = want.reshape(H, 64)
        elif k.split(".")[-1].startswith("x_"):
            want = want.reshape(1, 1, -1)
        assert g.shape == want.shape, k
        np.testing.assert_array_equal(g, want, err_msg=k)
    assert set(got) == {k for k in p if not (".v_lora_" in k and k.startswith("blocks.0."))}


def test_build_dense_weights_refusals(tmp_path):
    from swiftrwkv_amd import quant as Q
    path = str(tmp_path / "partial.rwkvq")
    w = (np.random.default_rng(0).standard_normal((256, 256)) * 0.02).astype(np.float32)
    Q.write_rwkvq(path, {"blocks.0.att.key.weight": Q.sb6_entry(w, 4, 4)}, n_layer=1, n_embd=256, vocab_size=512)
    with pytest.raises(Q.PartialExport):
        Q.RwkvqSidecar.from_rwkvq(path, device="cpu").build_dense_weights()
    path2 = str(tmp_path / "nolayers.rwkvq")
    Q.write_rwkvq(path2, {"ln_out.weight": ({"kind": "dense", "shape": [256]}, {"dense": np.ones(256, np.float16)})})
    with pytest.raises(Q.IncompleteManifest):
        Q.RwkvqSidecar.from_rwkvq(path2, device="cpu").build_dense_weights()


def file_projections(orc, T, shape):
    """fp64 dense matrices of the file's projections, dequantised by the
    oracle from the disk buffers."""
    W = {}
    for key, OUT, IN in shape.projections():
        m, f = T[key]
        if m["kind"] == "sb6":
            qblk, qsqm, ddm, xb = orc.sb6_to_k3(f["codes_packed"], f.get("gw_qh"), f.get("gw_qh2"), f["gw_qsqm"],
                                                f["gw_d"].view(np.uint16), f["gw_dm"].view(np.uint16), OUT, IN)
            W[key] = orc.sb6_dequant(qblk, qsqm, ddm, OUT, IN, xb).astype(np.float64)
        elif m["kind"] == "sym":
            W[key] = orc.sym_dequant(f["codes"].view(np.uint8), f["gw_qs"].view(np.uint8),
                                     f["gw_d"].view(np.uint16), OUT, IN, 8).astype(np.float64)
        else:
            W[key] = f["dense"].astype(np.float64)
    return W


def test_prefill_equals_sequence_and_steps():
    """The oracle's parallel pass (fp32 base, fp32 low-rank matrices, where
    `lin` has no narrowing either) equals the whole-sequence formulation's
    last logits and the token-by-token decode, states included; the fp16 base
    moves the logits by its roundings only (~1e-4)."""
    p = syn.x070_dense_params(TINY, seed=12, lora_dtype=np.float32)
    proj = syn.x070_projections(TINY, nthreads=4)
    W = X.dequant_projections(proj)
    ids = [5, 9, 300, 7, 100, 42]
    lg, st = X.prefill(p, W, ids, TINY.n_layer, TINY.n_head)
    seq = X.sequence(p, W, ids, TINY.n_layer, TINY.n_head)
    assert np.abs(lg - seq[-1]).max() <= 1e-12 * np.abs(seq).max()
    ost = X.State.zeros(TINY.n_layer, 1, TINY.n_head)
    for i in ids:
        step = X.step(p, W, [i], ost, TINY.n_layer, TINY.n_head)
    assert np.abs(lg - step[0]).max() <= 1e-12 * np.abs(step).max()
    for a, b in ((st.wkv, ost.wkv), (st.tmix_prev, ost.tmix_prev), (st.cmix_prev, ost.cmix_prev)):
        assert np.abs(a - b).max() <= 1e-12 * (np.abs(b).max() + 1)
    lg16, _ = X.prefill(p, W, ids, TINY.n_layer, TINY.n_head, f16_base=True)
    d = np.abs(lg16 - lg).max() / np.abs(lg).max()
    assert 1e-6 < d < 1e-2
