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
* rows of a batch are independent.
"""
import numpy as np
import pytest
import torch

from oracle import x070 as X
from swiftrwkv_amd import synthetic as syn

TINY = syn.X070Shape("tiny", 2, 256, 1024, vocab=512)


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
