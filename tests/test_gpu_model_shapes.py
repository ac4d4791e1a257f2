"""GPU parity at the full model widths: the decode GEMVs of the 0.4B
(D 1024, FFN 4096) and 7B-class (D 4096, FFN 14336) x070 shapes with the
65536-row head, the long-context WKV-7 prefill (B1 T8192 H64), the training
forward + backward over 256 checkpoint chunks (T 4096), and whole decode
tokens at the 1.5B and 7B-class widths — each against the fp64 oracle.

Tolerances (max|got − ref| / max|ref|): GEMV 2e-5 (RwkvqSb6GEMVTests.swift:53-77);
WKV forward / state / fp32 gradients 1e-5 (WKV7TrainKernelTests.swift:67-156
bounds 1e-3, the path's own 1e-5); gradients stored in bf16 1e-2; decode
tokens as in test_gpu_x070 (2e-5 with fp32 low-rank matrices, 5e-4 with fp16
ones, whose fp16 rounding points may flip by one ulp against fp64).
"""
import sys

import numpy as np
import pytest
import torch

from oracle import x070 as X
from swiftrwkv_amd import kernel as K, quant as Q, synthetic as syn
from swiftrwkv_amd.x070 import X070Decoder

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a, dt=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return t if dt is None else t.to(dt)


def host(t):
    return t.detach().float().cpu().numpy()


def rel(ref, got):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(ref - np.asarray(got, np.float64)).max() / (np.abs(ref).max() + 1e-30))


def random_k3(OUT, IN, rng):
    """A 4-bit sb6 matrix drawn directly in the K3 layout the kernels read:
    any byte is a pair of codes; qs in 0..63, stored qm − 31 in −31..32;
    fp16 super-block scales.  Dequant is a pure function of these bytes."""
    NB, NSB = IN // 32, IN // 256
    qblk = rng.integers(0, 256, (OUT, NB * 16), dtype=np.uint8)
    qsqm = np.empty((OUT, NB, 2), np.uint8)
    qsqm[..., 0] = rng.integers(0, 64, (OUT, NB), dtype=np.uint8)
    qsqm[..., 1] = rng.integers(-31, 33, (OUT, NB)).astype(np.int8).view(np.uint8)
    ddm = rng.uniform(1e-4, 3e-3, (OUT, NSB * 2)).astype(np.float16)
    return qblk, qsqm.reshape(OUT, NB * 2), ddm


GEMV_0B4 = [(1024, 1024), (4096, 1024), (1024, 4096), (65536, 1024)]
GEMV_7B = [(4096, 4096), (14336, 4096), (4096, 14336), (65536, 4096)]


@pytest.mark.parametrize("OUT,IN,N", [(o, i, n) for o, i in GEMV_0B4 for n in (1, 8, 32)] +
                         [(o, i, n) for o, i in GEMV_7B for n in (1, 16)])
def test_sb6_gemv_at_model_widths(orc, OUT, IN, N):
    case(f"sb6 gemv {OUT}x{IN} N={N}")
    rng = np.random.default_rng(OUT * 7 + IN)
    qblk, qsqm, ddm = random_k3(OUT, IN, rng)
    x = rng.standard_normal((N, IN)).astype(np.float32)
    y = Q.rwkvq_sb6_gemv(dev(x), dev(qblk), dev(qsqm), dev(ddm), OUT, IN, 0)
    want = orc.sb6_gemv_f64(x, qblk, qsqm, ddm.view(np.uint16), OUT, IN, 0)
    err = rel(want, host(y))
    print(f"[gemv] {OUT}x{IN} N={N}: rel {err:.2e}", flush=True)
    assert err < 2e-5


@pytest.mark.parametrize("N", [1, 16])
def test_fused_rkv_gemv_7b_width(orc, N):
    """r/k/v of a 4096-wide layer as one launch (3 × 4096 × 4096): row o of
    input n reads x[3n + o // 4096]."""
    case(f"fused sb6 r/k/v 3x4096x4096 N={N}")
    D = 4096
    rng = np.random.default_rng(41 + N)
    qblk, qsqm, ddm = random_k3(3 * D, D, rng)
    x = rng.standard_normal((N * 3, D)).astype(np.float32)
    y = Q.rwkvq_sb6_gemv(dev(x), dev(qblk), dev(qsqm), dev(ddm), 3 * D, D, 0, out_per=D)
    assert y.shape == (N, 3 * D)
    got = host(y)
    for m in range(3):
        rows = slice(m * D, (m + 1) * D)
        want = orc.sb6_gemv_f64(x[m::3], qblk[rows], qsqm[rows], ddm[rows].view(np.uint16), D, D, 0)
        err = rel(want, got[:, rows])
        assert err < 2e-5, m


def test_prefill_wkv_long_context(orc):
    """B1 T8192 H64 fp32, the 7B-class prefill layer (config-0 inputs)."""
    case("wkv7 seq fwd B1 T8192 H64")
    x = syn.wkv_inputs_config0(1, 8192, 64, seed=11)
    out, h = K.wkv7_sequence_forward(*[dev(z) for z in x])
    o64, h64 = orc.wkv7_fwd_f64(*x)
    eo, eh = rel(o64, host(out)), rel(h64, host(h))
    print(f"[wkv] T8192 H64: out {eo:.2e}, state {eh:.2e}", flush=True)
    assert eo < 1e-5 and eh < 1e-5


def _train(x, dt, g, h0=None, gh=None):
    ins = [dev(z, dt).requires_grad_(True) for z in x]
    hin = None if h0 is None else dev(h0).requires_grad_(True)
    o, h = K.wkv7_train_with_state(*ins, h_in=hin)
    loss = (o * dev(g)).sum()
    if gh is not None:
        loss = loss + (h * dev(gh)).sum()
    loss.backward()
    return o, h, [z.grad for z in ins] + ([hin.grad] if hin is not None else [])


def test_train_t4096_bf16_config0_inputs(orc):
    """256 checkpoint chunks of recompute-then-reverse, bf16 inputs and
    gradients (the training shape's precision), B1 H2."""
    case("train fwd+bwd bf16 B1 T4096 H2")
    x = [host(dev(z, torch.bfloat16)) for z in syn.wkv_inputs_config0(1, 4096, 2, seed=12)]
    g = np.random.default_rng(12).standard_normal((1, 4096, 2, 64)).astype(np.float32)
    o, h, grads = _train(x, torch.bfloat16, g)
    o64, h64 = orc.wkv7_fwd_f64(*x)
    eo, eh = rel(o64, host(o)), rel(h64, host(h))
    assert eo < 1e-5 and eh < 1e-5
    want = orc.wkv7_bwd_f64(*x, None, g, None)
    errs = [rel(w_, host(g_)) for w_, g_ in zip(want, grads)]
    print("[train] T4096 bf16 rel: " + ", ".join(f"{e:.1e}" for e in errs), flush=True)
    assert all(t.dtype == torch.bfloat16 for t in grads)
    assert max(errs) < 1e-2


def test_train_t1024_fp32_sixteen_row_layout(orc):
    """fp32, B2 T1024 H128 (B·H = 256: the sixteen-rows-per-wave forward),
    with an initial state and a final-state cotangent."""
    case("train fwd+bwd fp32 B2 T1024 H128")
    x = syn.wkv_inputs_train(2, 1024, 128, seed=13)
    h0 = syn.state(2, 128, scale=0.1, seed=113)
    rng = np.random.default_rng(13)
    g = rng.standard_normal((2, 1024, 128, 64)).astype(np.float32)
    gh = (rng.standard_normal((2, 128, 64, 64)) * 0.3).astype(np.float32)
    o, h, grads = _train(x, torch.float32, g, h0, gh)
    o64, h64 = orc.wkv7_fwd_f64(*x, h0)
    eo, eh = rel(o64, host(o)), rel(h64, host(h))
    assert eo < 1e-5 and eh < 1e-5
    want = orc.wkv7_bwd_f64(*x, h0, g, gh)
    errs = [rel(w_, host(g_)) for w_, g_ in zip(want, grads)]
    print("[train] T1024 H128 fp32 rel: " + ", ".join(f"{e:.1e}" for e in errs), flush=True)
    assert max(errs) < 1e-5


def _dequant_shared(proj):
    """fp64 matrices of projections whose layers share packed bytes, each
    distinct buffer dequantised once."""
    memo, W = {}, {}
    for k, q in proj.items():
        if id(q[0]) not in memo:
            memo[id(q[0])] = X.dequant_projections({k: q})[k]
        W[k] = memo[id(q[0])]
    return W


@pytest.mark.parametrize("shape,lora", [(syn.X070_1B5, "f32"), (syn.X070_1B5, "f16"),
                                        (syn.X070Shape("7B-class, 4 layers", 4, 4096, 14336), "f32")])
def test_decode_tokens_at_model_width(shape, lora):
    """Two decode tokens through every kernel of the step (1.5B: all 24
    layers; 7B-class: four layers of the full width, the 14336-wide FFN and the
    65536-row head).  Layers share their packed projection bytes (distinct
    dense parameters per layer)."""
    case(f"decode {shape.name} low-rank {lora}")
    proj = syn.x070_projections(shape, nthreads=16, share_layers=True)
    W = _dequant_shared(proj)
    p = syn.x070_dense_params(shape, seed=21, lora_dtype=np.float32 if lora == "f32" else np.float16)
    d = X070Decoder(shape.n_layer, shape.n_embd, shape.ffn, shape.vocab, p, proj, DEV)
    st = d.new_state(1)
    ost = X.State.zeros(shape.n_layer, 1, shape.n_head)
    tol = 2e-5 if lora == "f32" else 5e-4
    for t, i in enumerate((17, 60000)):
        got = d.step([i], st).cpu().numpy()
        ref = X.step(p, W, [i], ost, shape.n_layer, shape.n_head)
        err = rel(ref, got)
        print(f"[x070] {shape.name} low-rank {lora} token {t}: rel {err:.3e}", flush=True)
        assert err < tol, t
    e_state = rel(ost.wkv, host(st.wkv))
    print(f"[x070] {shape.name} low-rank {lora} WKV states after 2 tokens: rel {e_state:.3e}", flush=True)
    assert e_state < tol
