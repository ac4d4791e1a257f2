"""GPU parity at the full sizes of the three workloads the other files check
in parts:

* WKV-7 training forward + backward at B8 T4096 H32 with bf16 inputs and
  gradients (the 1.5B training shape, B·H = 256: the sixteen-rows-per-wave
  forward and the column-owned backward over 256 checkpoint chunks).  Every
  (batch, head) pair is an independent recurrence, so four (b, h) slices
  compared with the fp64 oracle run on those slices alone are exact checks of
  the full launch; the whole tensors are checked by properties (finite,
  deterministic, keep == recompute).
* Batched decode of the 0.4B shape at its full depth (24 layers, n_embd 1024,
  H 16) at batch 8 and 32: two steps of every row against the fp64 oracle.
* The 7B-class width (n_embd 4096, H 64, FFN 14336, the 65536-row head; four
  layers sharing packed bytes): the parallel prefill of a 1024-token and a
  700-token prompt on the fp16 long pass with the time-chunked WKV-7, and two
  decode steps at batch 16.

Tolerances (max|got − ref| / max|ref|): WKV outputs, states and fp32
gradients 1e-5, bf16 gradients 1e-2 (WKV7TrainKernelTests.swift:67-156);
decode steps 2e-5 with fp32 low-rank matrices, as at the other widths;
fp16-base prefill 2e-3 (the fp16 rounding points of the long pass, as in
test_gpu_prefill).
"""
import sys

import numpy as np
import pytest
import torch

from oracle import x070 as X
from swiftrwkv_amd import _lib, kernel as K, synthetic as syn
from swiftrwkv_amd.x070 import X070Decoder, wkv_chunked_prefers

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def rel(ref, got):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(ref - np.asarray(got, np.float64)).max() / (np.abs(ref).max() + 1e-30))


def host(t):
    return t.detach().float().cpu().numpy()


def _dequant_shared(proj):
    memo, W = {}, {}
    for k, q in proj.items():
        if id(q[0]) not in memo:
            memo[id(q[0])] = X.dequant_projections({k: q})[k]
        W[k] = memo[id(q[0])]
    return W


# ───────────────────────── training, B8 T4096 H32 bf16 ─────────────────────────

SLICES = [(0, 0), (3, 17), (5, 31), (7, 8)]


def _train_full(xb, dy, dhT, keep):
    K.wkv7_keep_forward_outputs = keep
    try:
        ins = [z.clone().requires_grad_(True) for z in xb]
        h0 = torch.zeros((8, 32, 64, 64), device=DEV, requires_grad=True)
        o, h = K.wkv7_train_with_state(*ins, h_in=h0)
        loss = (o * dy).sum()
        if dhT is not None:
            loss = loss + (h * dhT).sum()
        loss.backward()
    finally:
        K.wkv7_keep_forward_outputs = True
    torch.cuda.synchronize()
    return o.detach(), h.detach(), [z.grad for z in ins] + [h0.grad]


@pytest.mark.parametrize("with_dhT", [False, True])
def test_train_b8_t4096_h32_bf16_full_size(orc, with_dhT):
    case(f"train fwd+bwd B8 T4096 H32 bf16, d_hT {'N(0,1)*0.3' if with_dhT else 'zero'}")
    B, T, H = 8, 4096, 32
    xs = syn.wkv_inputs_config0(B, T, H, seed=3)
    xb = [torch.from_numpy(z).to(DEV).to(torch.bfloat16) for z in xs]
    del xs
    rng = np.random.default_rng(3)
    dy_h = rng.standard_normal((B, T, H, 64), dtype=np.float32)
    dh_h = (rng.standard_normal((B, H, 64, 64), dtype=np.float32) * np.float32(0.3)) if with_dhT else None
    dy = torch.from_numpy(dy_h).to(DEV)
    dhT = None if dh_h is None else torch.from_numpy(dh_h).to(DEV)
    o, h, grads = _train_full(xb, dy, dhT, keep=True)
    assert o.dtype == torch.float32 and h.dtype == torch.float32
    assert all(g.dtype == torch.bfloat16 for g in grads[:6]) and grads[6].dtype == torch.float32
    for t in [o, h] + grads:
        assert bool(torch.isfinite(t).all())
    # each (b, h) is its own recurrence: the slices against the fp64 oracle
    x_host = [host(z) for z in xb]   # the bf16 values, widened exactly
    for b, hh in SLICES:
        sl = [np.ascontiguousarray(z[b:b + 1, :, hh:hh + 1]) for z in x_host]
        g_sl = np.ascontiguousarray(dy_h[b:b + 1, :, hh:hh + 1])
        gh_sl = None if dh_h is None else np.ascontiguousarray(dh_h[b:b + 1, hh:hh + 1])
        o64, h64 = orc.wkv7_fwd_f64(*sl)
        eo = rel(o64, host(o[b:b + 1, :, hh:hh + 1]))
        eh = rel(h64, host(h[b:b + 1, hh:hh + 1]))
        want = orc.wkv7_bwd_f64(*sl, np.zeros((1, 1, 64, 64), np.float32), g_sl, gh_sl)
        got = [host(g[b:b + 1, :, hh:hh + 1]) for g in grads[:6]] + [host(grads[6][b:b + 1, hh:hh + 1])]
        errs = [rel(w_, g_) for w_, g_ in zip(want, got)]
        print(f"[train] slice b{b} h{hh}: out {eo:.1e} state {eh:.1e} grads "
              + ", ".join(f"{e:.1e}" for e in errs), flush=True)
        assert eo < 1e-5 and eh < 1e-5, (b, hh)
        assert max(errs[:6]) < 1e-2, (b, hh)   # stored in bf16
        assert errs[6] < 1e-5, (b, hh)         # d(initial state), fp32
    # the whole launch: deterministic, and the recomputing forward gives the same bits
    o2, h2, grads2 = _train_full(xb, dy, dhT, keep=True)
    assert torch.equal(o, o2) and torch.equal(h, h2)
    assert all(torch.equal(p, q) for p, q in zip(grads, grads2))
    del o2, h2, grads2
    n = K.wkv7_train_forward_launches()
    o3, h3, grads3 = _train_full(xb, dy, dhT, keep=False)
    assert K.wkv7_train_forward_launches() - n == 2
    assert torch.equal(o, o3) and torch.equal(h, h3)
    assert all(torch.equal(p, q) for p, q in zip(grads, grads3))


# ───────────────────────── batched decode, 0.4B at full depth ─────────────────────────

@pytest.fixture(scope="module")
def model_0b4():
    proj = syn.x070_projections(syn.X070_0B4, nthreads=16, share_layers=True)
    return proj, _dequant_shared(proj)


@pytest.mark.parametrize("N", [8, 32])
def test_step_batch_0b4_full_depth(model_0b4, N):
    shape = syn.X070_0B4
    case(f"step_batch {shape.name} 24 layers batch {N}")
    proj, W = model_0b4
    p = syn.x070_dense_params(shape, seed=40 + N, lora_dtype=np.float32)
    d = X070Decoder(shape.n_layer, shape.n_embd, shape.ffn, shape.vocab, p, proj, DEV)
    st = d.new_state(N)
    ost = X.State.zeros(shape.n_layer, N, shape.n_head)
    rng = np.random.default_rng(N)
    for t in range(2):
        ids = [int(i) for i in rng.integers(0, shape.vocab, N)]
        got = d.step_batch(ids, st).cpu().numpy()
        ref = X.step(p, W, ids, ost, shape.n_layer, shape.n_head)
        err = max(rel(ref[i], got[i]) for i in range(N))
        print(f"[x070] {shape.name} batch {N} token {t}: worst row rel {err:.3e}", flush=True)
        assert err < 2e-5, t
    e_state = max(rel(ost.wkv[:, i], host(st.wkv[:, i])) for i in range(N))
    print(f"[x070] {shape.name} batch {N} WKV states after 2 tokens: worst row rel {e_state:.3e}", flush=True)
    assert e_state < 2e-5


# ───────────────────────── 7B-class width: prefill and batch-16 decode ─────────────────────────

SHAPE_7B4 = syn.X070Shape("7B-class width, 4 layers", 4, 4096, 14336)


@pytest.fixture(scope="module")
def model_7b4():
    proj = syn.x070_projections(SHAPE_7B4, nthreads=16, share_layers=True)
    return proj, _dequant_shared(proj)


def test_prefill_7b_width_chunked_wkv_fp16_base(model_7b4):
    shape = SHAPE_7B4
    case(f"prefill_batch {shape.name}, prompts of 1024 and 700 tokens, fp16 base, chunked WKV")
    proj, W = model_7b4
    p = syn.x070_dense_params(shape, seed=51, lora_dtype=np.float16)
    d = X070Decoder(shape.n_layer, shape.n_embd, shape.ffn, shape.vocab, p, proj, DEV)
    rng = np.random.default_rng(51)
    prompts = [[int(t) for t in rng.integers(0, shape.vocab, n)] for n in (1024, 700)]
    assert wkv_chunked_prefers(len(prompts), 1024, shape.n_head)
    n_ch, n_gemm = _lib.counters()["seq_chunked"], _lib.counters()["sb6_gemm"]
    logits, st = d.prefill_batch(prompts, base_dtype=torch.float16)
    torch.cuda.synchronize()
    assert _lib.counters()["seq_chunked"] - n_ch == shape.n_layer
    assert _lib.counters()["sb6_gemm"] - n_gemm == shape.n_layer * 4
    for i, pr in enumerate(prompts):
        ref, ost = X.prefill(p, W, pr, shape.n_layer, shape.n_head, f16_base=True)
        e = rel(ref, logits[i].cpu().numpy())
        ew = rel(ost.wkv[:, 0], host(st.wkv[:, i]))
        es = max(rel(ost.tmix_prev[:, 0], host(st.tmix_prev[:, i])),
                 rel(ost.cmix_prev[:, 0], host(st.cmix_prev[:, i])))
        print(f"[prefill] {shape.name} row {i} (T={len(pr)}): logits {e:.2e}, wkv {ew:.2e}, shift {es:.2e}",
              flush=True)
        assert e < 2e-3 and ew < 2e-3 and es < 2e-3, i


def test_step_batch_7b_width_batch16(model_7b4):
    shape = SHAPE_7B4
    N = 16
    case(f"step_batch {shape.name} batch {N}")
    proj, W = model_7b4
    p = syn.x070_dense_params(shape, seed=52, lora_dtype=np.float32)
    d = X070Decoder(shape.n_layer, shape.n_embd, shape.ffn, shape.vocab, p, proj, DEV)
    st = d.new_state(N)
    ost = X.State.zeros(shape.n_layer, N, shape.n_head)
    rng = np.random.default_rng(52)
    for t in range(2):
        ids = [int(i) for i in rng.integers(0, shape.vocab, N)]
        got = d.step_batch(ids, st).cpu().numpy()
        ref = X.step(p, W, ids, ost, shape.n_layer, shape.n_head)
        err = max(rel(ref[i], got[i]) for i in range(N))
        print(f"[x070] {shape.name} batch {N} token {t}: worst row rel {err:.3e}", flush=True)
        assert err < 2e-5, t
    e_state = max(rel(ost.wkv[:, i], host(st.wkv[:, i])) for i in range(N))
    print(f"[x070] {shape.name} batch {N} WKV states after 2 tokens: worst row rel {e_state:.3e}", flush=True)
    assert e_state < 2e-5
