"""Benchmark of the MI355X WKV-7 + .rwkvq hot path (one GPU).

Headline (`value`): "1.5B decode tok/s" — one-token decode of the 1.5B x070
shape (24 layers, n_embd 2048, FFN 8192, vocab 65536), batch 1, through the
whole step (X070Decoder.launch: embedding row + ln0; per layer ln1 / token
shift / lerps, the fused r/k/v GEMV with the low-rank first layers, the tmix
core with the WKV-7 step and tail, o_proj + residual, ln2 / shift, ffn key
relu², ffn value + residual; ln_out, head) captured in one HIP graph.  Weights
are sb6 4-bit encoded from seeded N(0, 0.02): 776 MB of packed projections
per token (> the 256 MB MALL), resident in HBM before the timed region.

`roofline` is for the token's GEMV-bearing launches (the r/k/v + low-rank,
o_proj, ffn key and ffn value launches of every layer and the head: ~86 % of
its kernel time): their algorithmic bytes (packed projections, the fp16
low-rank inner matrices, the fp32 rows they read and write) over their
average duration, measured live on a graph of the same step with its tmix
cores and layer norms left out, so those launches run back to back in step
order; `roofline.whole_token` is the whole token's algorithmic bytes over the
headline's time per token.  `cpu_baseline` times the
oracle's restatement of the reference's non-kernel decode path (dequantise
to fp32, x·Wᵀ per projection; MLX-op WKV step) on a bounded sample of 1.5B
tokens, checked against the GPU head GEMV first.

Also reported (`extra`): the 0.1B decode (GEMV + WKV chain of one token, and
the whole step), WKV-7 forward tokens/s at B1 T1024 H12 fp32, forward and
forward+backward at B8 T4096 H32 bf16 (checkpointed), the head-GEMV HBM GB/s,
batched decode of the 0.1B and 0.4B shapes (batch 1 / 8 / 32) and of the 1.5B
shape (batch 16), decode of the
7B-class shape (32 layers, n_embd 4096, FFN 14336) at batch 1 and 16, the
WKV-7 forward of one 7B-class prefill layer (B1 T8192 H64 fp32), and the CPU
restatements.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "WKV-7 tokens/s (fwd, fwd+bwd); .rwkvq GEMV GB/s; 1.5B decode tok/s"
HBM_PEAK_GBPS = 8000.0
# HBM bytes per launch of the head GEMV from two rocprofv3 counter passes
# (FETCH_SIZE, WRITE_SIZE) over `bench.py --mode kernels`, calibrated against a
# 256 MiB device copy; see profiles/hbm_traffic_decode_gemv_and_wkv7.md.
HEAD_GEMV_TRAFFIC_BYTES = 29494797
# The same for the average GEMV launch of one 0.1B decode token (eager tokens
# over rotated weight copies); same profile.
DECODE_GEMV_TRAFFIC_BYTES = 1744043
# The same for the average GEMV launch of one 1.5B decode token (582 launches
# of 6 eager tokens; profiles/hbm_traffic_decode_1.5B_gemv.md).
DECODE_1B5_GEMV_TRAFFIC_BYTES = 8291062
# The same for the average GEMV-bearing launch of the 1.5B x070 step (per layer
# the r/k/v + low-rank, o_proj, ffn key and ffn value launches, and the head);
# profiles/counters_decode_1.5B_step.md.
DECODE_1B5_STEP_GEMV_TRAFFIC_BYTES = 9027701
VALU_PEAK_TFLOPS = 157.3


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--copies", type=int, default=6)
    p.add_argument("--skip-cpu", action="store_true")
    p.add_argument("--skip-wkv", action="store_true")
    p.add_argument("--skip-more", action="store_true", help="skip batched / 7B-class decode and the prefill pass")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--mode", choices=["bench", "kernels", "e2e", "batch", "step", "prefill", "prefill_short"], default="bench",
                   help="kernels: run each dominant kernel alone (for rocprofv3 counter passes); "
                        "e2e / batch: x070 decode tokens / batched GEMV + WKV decode steps only (for kernel traces); "
                        "step: the 1.5B headline step alone (eager tokens, then graph replays; counter passes); "
                        "prefill: two passes of the 7B-class T8192 prefill (kernel traces)")
    return p.parse_args()


def kernel_ms(launch, stream=None) -> float:
    """Duration of the single library kernel `launch()` enqueues, timed by the
    kernel's own start / stop timestamps (rwkv_time_next_launch)."""
    import torch
    from swiftrwkv_amd import _lib

    stream = stream or torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    e1.record(stream)
    _lib.call("rwkv_time_next_launch", e0.cuda_event, e1.cuda_event)
    launch()
    e1.synchronize()
    return e0.elapsed_time(e1)


# MFMA issues of the chunk-transform kernel per 32-token chunk of one head:
# 216 per wave × 4 waves + 8 for T21 (wkv7_chunk_prep_kernel), each
# v_mfma_f32_16x16x4_f32 = 2048 flops.
CHUNK_PREP_MFMA_FLOPS = (216 * 4 + 8) * 2048
FP32_MFMA_PEAK_TFLOPS = 157.3


def graph_ms(launch, reps=20) -> float:
    """Average replay time of a HIP graph holding `launch()`'s kernels (no
    host overhead between them)."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        launch()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / reps


def bench_wkv_chunked(dev, B, T, H, gen, reps=10):
    """The time-chunked WKV-7 forward (rwkv_wkv7_seq_fwd_chunked) next to the
    step-by-step one on the same inputs: the call's two launches replayed from
    a HIP graph, the chunk-transform kernel alone (its own timestamps) with
    its matrix-core roofline, and the step kernel alone."""
    import torch
    from swiftrwkv_amd import _lib, kernel as K

    x = [torch.from_numpy(z).to(dev) for z in gen(B, T, H, seed=0)]
    ws = torch.empty(K.wkv7_chunked_workspace_bytes(B, T, H), dtype=torch.uint8, device=dev)
    out = torch.empty((B, T, H, 64), device=dev)
    h = torch.empty((B, H, 64, 64), device=dev)
    ptrs = [z.data_ptr() for z in x]

    def chunked():
        _lib.call("rwkv_wkv7_seq_fwd_chunked", *ptrs, _lib.F32, None, out.data_ptr(), h.data_ptr(), B, T, H,
                  ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)

    def step():
        _lib.call("rwkv_wkv7_seq_fwd", *ptrs, _lib.F32, None, out.data_ptr(), h.data_ptr(), B, T, H,
                  torch.cuda.current_stream().cuda_stream)

    ms = graph_ms(chunked, reps)
    prep_ms = sum(kernel_ms(chunked) for _ in range(reps)) / reps
    step_ms = sum(kernel_ms(step) for _ in range(reps)) / reps
    n_chunks = B * H * ((T + 31) // 32)
    flops = n_chunks * CHUNK_PREP_MFMA_FLOPS
    del x, ws, out, h
    torch.cuda.empty_cache()
    return {"ms": ms, "tok_s": B * T / (ms * 1e-3), "step_kernel_ms": step_ms, "speedup_vs_step": step_ms / ms,
            "chunk_prep_ms": prep_ms, "scan_ms": ms - prep_ms,
            "chunk_prep_mfma_tflops": flops / (prep_ms * 1e-3) / 1e12,
            "chunk_prep_mfma_frac": flops / (prep_ms * 1e-3) / (FP32_MFMA_PEAK_TFLOPS * 1e12)}


# ───────────────────────────── decode model ─────────────────────────────

class DecodeModel:
    """Packed weights of all projections (K3 layout on the device), per copy."""

    def __init__(self, shape, copies, dev, nthreads, only=None, share_layers=False):
        import numpy as np
        import torch
        from swiftrwkv_amd import quant as Q

        self.shape = shape
        self.host = {}
        self.dev = [dict() for _ in range(copies)]
        self.bytes_per_token = 0
        t0 = time.time()
        for idx, (key, OUT, IN) in enumerate(shape.projections()):
            if only is not None and key not in only:
                continue
            parts = key.split(".")
            if share_layers and parts[0] == "blocks" and parts[1] != "0":
                # same packed bytes as layer 0's matrix, in its own device buffer
                self.host[key] = self.host[".".join(["blocks", "0"] + parts[2:])]
            else:
                rng = np.random.default_rng(1000 + idx)
                w = (rng.standard_normal((OUT, IN), dtype=np.float32) * np.float32(0.02))
                disk = Q.encode_sb6(w, 4, nthreads)
                qblk, qsqm, ddm, xb = Q.rwkvq_sb6_to_k3(disk["codes_packed"], disk["gw_qsqm"], disk["gw_d"],
                                                        disk["gw_dm"], None, None, (OUT, IN))
                self.host[key] = (qblk, qsqm, ddm, OUT, IN)
            qblk, qsqm, ddm = self.host[key][:3]
            self.bytes_per_token += qblk.nbytes + qsqm.nbytes + ddm.nbytes + 4 * (IN + OUT)
        self.launches_per_token = 0
        # device buffers; r/k/v of a layer row-concatenated (one fused launch)
        groups = {}
        for key in self.host:
            if ".att.receptance." in key or ".att.key." in key or ".att.value." in key:
                groups.setdefault(key.split(".att.")[0] + ".att.rkv", []).append(key)
            else:
                groups[key] = [key]
        for gkey, members in groups.items():
            parts = [self.host[m] for m in members]
            base = (torch.from_numpy(np.concatenate([p[0] for p in parts])).to(dev),
                    torch.from_numpy(np.concatenate([p[1] for p in parts])).to(dev),
                    torch.from_numpy(np.concatenate([p[2] for p in parts]).view(np.float16)).to(dev))
            self.dev[0][gkey] = base
            for c in range(1, copies):
                self.dev[c][gkey] = tuple(z.clone() for z in base)
        self.launches_per_token = len(groups)
        log(f"encoded {len(self.host)} matrices of {shape.name} in {time.time() - t0:.1f}s, "
            f"{self.bytes_per_token / 1e6:.1f} MB per token, {copies} device copies")


class DecodeStep:
    """Buffers and the launch sequence of one decode token (batch B)."""

    def __init__(self, model: DecodeModel, dev, B=1, seed=0):
        import numpy as np
        import torch
        from swiftrwkv_amd import synthetic as syn

        s = model.shape
        self.model, self.B, self.L, self.H, self.D, self.F = model, B, s.n_layer, s.n_head, s.n_embd, s.ffn
        rng = np.random.default_rng(seed)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
        self.xD = t(rng.standard_normal((B, self.D)))
        self.xrkv = t(rng.standard_normal((B * 3, self.D)))   # token-shifted r/k/v inputs, per row
        self.xF = t(np.maximum(rng.standard_normal((B, self.F)), 0) ** 2 * 0.1)
        self.y_rkv = torch.empty((B, 3 * self.D), device=dev)
        self.y_o = torch.empty((B, self.D), device=dev)
        self.y_k = torch.empty((B, self.F), device=dev)
        self.y_v = torch.empty((B, self.D), device=dev)
        self.logits = torch.empty((B, s.vocab), device=dev)
        self.wkv = torch.empty((B, self.H, 64), device=dev)
        self.tail = torch.empty((B, self.D), device=dev)
        vec = syn.wkv_inputs_config0(self.L, B, self.H, seed=seed + 1)   # [L, B, H, 64] per input
        self.rwkvab = [t(z) for z in vec]
        self.state = torch.zeros((self.L, B, self.H, 64, 64), device=dev)
        self.rk = t(rng.standard_normal((self.L, self.D)) * 0.1)
        self.lnw = t(rng.standard_normal((self.L, self.D)) * 0.5 + 1)
        self.lnb = t(rng.standard_normal((self.L, self.D)) * 0.1)
        self.g = t(rng.standard_normal((self.L, B, self.D)))
        # batches of 8-32 rows take the matrix-core batched GEMV (one
        # workspace for all projections: the launches run in stream order)
        from swiftrwkv_amd import _lib, quant as Q
        L = _lib.lib()
        self.mfma, need = set(), 0
        D, F = self.D, self.F
        for OUT, IN, per in ((3 * D, D, D), (D, D, D), (F, D, F), (D, F, D), (s.vocab, D, s.vocab)):
            if B <= 32 and Q.rwkvq_sb6_gemv_batch_prefers(B, OUT, IN) and \
                    L.rwkv_sb6_gemv_batch_applies(B, OUT, IN, 0, per):
                self.mfma.add((OUT, IN, per))
                need = max(need, int(L.rwkv_sb6_gemv_batch_workspace(B, OUT, IN, per)))
        self.ws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
        # their weights in the matrix cores' T16 order, one copy per device copy
        self.t16 = [{} for _ in model.dev]
        if self.mfma:
            for c, W in enumerate(model.dev):
                for key, q in W.items():
                    OUT, IN = q[0].shape[0], q[0].shape[1] * 2   # qblk [OUT, IN/2]
                    per = D if key.endswith("att.rkv") else OUT
                    if (OUT, IN, per) in self.mfma:
                        self.t16[c][id(q)] = Q.rwkvq_sb6_t16(q[0], q[1], q[2], OUT, IN)

    def _gemv(self, L, x, q, y, OUT, IN, per, stream, fused=False, copy=0):
        from swiftrwkv_amd import _lib
        if (OUT, IN, per) in self.mfma:
            t = self.t16[copy][id(q)]
            _lib.check(L.rwkv_sb6_gemv_batch_t16(x.data_ptr(), self.B, t[0].data_ptr(), t[1].data_ptr(),
                                                 t[2].data_ptr(), y.data_ptr(), OUT, IN, per, 0, self.ws.data_ptr(),
                                                 self.ws.numel(), stream))
        elif fused:
            _lib.check(L.rwkv_sb6_gemv_fused(x.data_ptr(), self.B, q[0].data_ptr(), q[1].data_ptr(), q[2].data_ptr(),
                                             y.data_ptr(), OUT, IN, 0, per, stream))
        else:
            _lib.check(L.rwkv_sb6_gemv(x.data_ptr(), self.B, q[0].data_ptr(), q[1].data_ptr(), q[2].data_ptr(),
                                       y.data_ptr(), OUT, IN, 0, stream))

    def launch(self, copy: int, stream: int, gemv_only=False):
        """Enqueue one token (`gemv_only`: its GEMV launches alone)."""
        from swiftrwkv_amd import _lib
        L = _lib.lib()
        W = self.model.dev[copy]
        B, D, F, H = self.B, self.D, self.F, self.H

        def gemv(x, key, y):
            OUT, IN = self.model.host[key][3], self.model.host[key][4]
            self._gemv(L, x, W[key], y, OUT, IN, OUT, stream, copy=copy)

        for l in range(self.L):
            # r/k/v in one launch, x rows (x_r, x_k, x_v) per token
            self._gemv(L, self.xrkv, W[f"blocks.{l}.att.rkv"], self.y_rkv, 3 * D, D, D, stream, fused=True,
                       copy=copy)
            if gemv_only:
                gemv(self.tail, f"blocks.{l}.att.output.weight", self.y_o)
                gemv(self.xD, f"blocks.{l}.ffn.key.weight", self.y_k)
                gemv(self.xF, f"blocks.{l}.ffn.value.weight", self.y_v)
                continue
            r, w, k, v, a, b = (z[l] for z in self.rwkvab)
            st = self.state[l]
            _lib.check(L.rwkv_wkv7_step_tail(r.data_ptr(), w.data_ptr(), k.data_ptr(), v.data_ptr(), a.data_ptr(),
                                             b.data_ptr(), st.data_ptr(), st.data_ptr(), self.rk[l].data_ptr(),
                                             self.lnw[l].data_ptr(), self.lnb[l].data_ptr(), self.g[l].data_ptr(),
                                             None, self.tail.data_ptr(), B, H, float(64e-5), stream))
            gemv(self.tail, f"blocks.{l}.att.output.weight", self.y_o)
            gemv(self.xD, f"blocks.{l}.ffn.key.weight", self.y_k)
            gemv(self.xF, f"blocks.{l}.ffn.value.weight", self.y_v)
        gemv(self.xD, "head.weight", self.logits)


def run_decode(model, dev, B, steps, warmup, copies, verify=True):
    """One decode token per HIP graph replay (one graph per weight copy);
    returns (wall seconds, GPU ms) over `steps` tokens of batch B."""
    import torch

    step = DecodeStep(model, dev, B=B)
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        s0 = step.state.clone()
        if verify:   # eager reference token from a known state
            step.launch(0, stream.cuda_stream)
            eager = step.logits.clone()
            eager_state = step.state.clone()
            torch.cuda.synchronize()
        graphs = []
        for c in range(copies):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                step.launch(c, torch.cuda.current_stream().cuda_stream)
            graphs.append(g)
        torch.cuda.synchronize()
        if verify:
            for rep in range(3):   # every replay reproduces the eager token bitwise
                step.state.copy_(s0)
                torch.cuda.synchronize()
                graphs[rep % copies].replay()
                torch.cuda.synchronize()
                if not (torch.equal(step.logits, eager) and torch.equal(step.state, eager_state)):
                    raise RuntimeError(f"graph replay {rep} differs from the eager decode token")
        step.state.copy_(s0)
        for i in range(warmup):
            graphs[i % copies].replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for i in range(steps):
            graphs[i % copies].replay()
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    return step, wall, e0.elapsed_time(e1)


def run_x070(model, dev, steps, warmup, copies=1, B=1):
    """End-to-end x070 decode token (X070Decoder: embedding + ln0, per layer
    ln1 / shift / lerps, fused r/k/v GEMV, low-rank branches, tmix core with
    the WKV step and tail, o_proj + residual, ln2 / shift, ffn key relu², ffn
    value + residual; ln_out, head) over `model`'s packed projections, one
    HIP graph per weight copy; returns (wall s, GPU ms, launches per token)
    over `steps` tokens of B rows."""
    import torch
    from swiftrwkv_amd import synthetic as syn
    from swiftrwkv_amd.x070 import X070Decoder

    s = model.shape
    dense = syn.x070_dense_params(s, seed=11)
    decs = [X070Decoder(s.n_layer, s.n_embd, s.ffn, s.vocab, dense, model.host, dev) for _ in range(copies)]
    st = decs[0].new_state(B)
    ids = torch.randint(0, s.vocab, (B,), dtype=torch.int32, device=dev)
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        for d in decs:
            d.launch(ids, st)   # buffers exist before capture; the state is not zero
        torch.cuda.synchronize()
        s0 = st.clone()
        eager = decs[0].launch(ids, st).clone()
        eager_wkv = st.wkv.clone()
        graphs = []
        for d in decs:
            st.copy_(s0)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                out = d.launch(ids, st)
            graphs.append((g, out))
        torch.cuda.synchronize()
        st.copy_(s0)
        torch.cuda.synchronize()
        graphs[0][0].replay()
        torch.cuda.synchronize()
        if not (torch.equal(graphs[0][1], eager) and torch.equal(st.wkv, eager_wkv)):
            raise RuntimeError("x070 decode graph replay differs from the eager token")
        for i in range(warmup):
            graphs[i % copies][0].replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for i in range(steps):
            graphs[i % copies][0].replay()
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    launches = decs[0].launches_per_token(B)
    del decs, graphs
    torch.cuda.empty_cache()
    return wall, e0.elapsed_time(e1), launches


def x070_step_bytes(dec):
    """Algorithmic bytes of one batch-1 token of the row-forming x070 step
    (X070Decoder._layer_ln_fused): (bytes of its GEMV-bearing launches,
    bytes of the whole token).  Each buffer counts once per launch that must
    read or write it: packed projections (K3 bytes), the fp16 low-rank
    matrices, the fp32 rows (activations, layer-norm and lerp parameters,
    shift rows) and the WKV state (read and written)."""
    D, F, V, H = dec.D, dec.F, dec.V, dec.H
    packed = lambda key: sum(int(b.numel()) * b.element_size() for b in dec.proj[key].bufs)
    rw, ra, rv, rg = dec.ranks
    gemv = whole = 0
    for l in range(dec.L):
        RT = rw + ra + rg + (rv if l > 0 else 0)
        lora = RT * D * 2   # the branch matrices' inner (A) rows, fp16
        # r/k/v + low-rank inner products: x, prev, 6 lerp rows, ln1 w/b in; y_rkv, la, xl1 out
        rkv = packed(f"blocks.{l}.att.rkv") + lora + 4 * (10 * D + 3 * D + RT + D)
        o = packed(f"blocks.{l}.att.output.weight") + 4 * (D + 2 * D)   # tout in; x read and written
        # ffn key: x, prev, lerp row, ln2 w/b in; hk, xl2 out
        key = packed(f"blocks.{l}.ffn.key.weight") + 4 * (5 * D + F + D)
        # ffn value: hk in; x read and written; the shift row copied
        val = packed(f"blocks.{l}.ffn.value.weight") + 4 * (F + 2 * D + 2 * D)
        # tmix core: the branch matrices' outer (B) rows, y_rkv, la, per-head
        # vectors (3 biases, k_k, k_a, r_k, ln_x w/b, v_first), the state twice, tout
        core = lora + 4 * (3 * D + RT + 9 * D + 2 * H * 64 * 64 + D)
        gemv += rkv + o + key + val
        whole += rkv + o + key + val + core
    head = packed("head.weight") + 4 * (D + V)
    lnio = 2 * 4 * (3 * D) + 2 * D   # emb row (fp16) + ln0, ln_out: row, w, b in, row out
    return gemv + head, whole + head + lnio


class _SkipLaunches:
    """The library with some entry points turned into no-ops (they return
    RWKV_OK without launching): a graph captured through it holds the
    other launches of a step, in the step's order."""

    # the entry points that launch a GEMV-bearing kernel (one launch each here)
    LAUNCHES = {"rwkv_x070_rkv_lora_ln", "rwkv_x070_ffn_key_ln", "rwkv_x070_ffn_value", "rwkv_x070_rkv_lora",
                "rwkv_sb6_gemv_ep", "rwkv_sb6_gemv_fused", "rwkv_sb6_gemv"}

    def __init__(self, lib, skip):
        self._lib, self._skip, self.kept = lib, set(skip), 0

    def __getattr__(self, name):
        f = getattr(self._lib, name)
        if name in self._skip:
            return lambda *a: 0
        if name in self.LAUNCHES:
            def counted(*a):
                self.kept += 1
                return f(*a)
            return counted
        return f


def bench_step_gemv_launches(model, dev, reps=100):
    """In-step roofline of the 1.5B token's GEMV-bearing launches: the
    X070Decoder step captured with its tmix cores and layer norms left out
    (r/k/v + low-rank, o_proj + residual, ffn key, ffn value + residual per
    layer, and the head: the step's own kernels, grids and bytes, back to back
    in step order), replayed; returns (algorithmic bytes of those launches,
    launches, average ms per launch, whole-token bytes)."""
    import torch
    from swiftrwkv_amd import _lib, synthetic as syn
    from swiftrwkv_amd.x070 import X070Decoder

    s = model.shape
    dense = syn.x070_dense_params(s, seed=11)
    dec = X070Decoder(s.n_layer, s.n_embd, s.ffn, s.vocab, dense, model.host, dev)
    st = dec.new_state(1)
    ids = torch.randint(0, s.vocab, (1,), dtype=torch.int32, device=dev)
    stream = torch.cuda.Stream(device=dev)
    lib = _lib.lib
    proxy = _SkipLaunches(lib(), {"rwkv_x070_tmix_core", "rwkv_layer_norm"})
    with torch.cuda.stream(stream):
        dec.launch(ids, st)   # buffers exist before capture
        torch.cuda.synchronize()
        _lib.lib = lambda: proxy
        try:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                dec.launch(ids, st)
        finally:
            _lib.lib = lib
        n = proxy.kept
        for _ in range(5):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
    gemv_bytes, whole_bytes = x070_step_bytes(dec)
    del dec, g
    torch.cuda.empty_cache()
    return gemv_bytes, n, e0.elapsed_time(e1) / (reps * n), whole_bytes


def x070_line(model, dev, steps, warmup, copies=1, B=1):
    wall, gpu_ms, launches = run_x070(model, dev, steps, warmup, copies, B)
    ms = wall * 1e3 / steps
    log(f"x070 decode e2e {model.shape.name} batch {B}: {ms:.3f} ms per token ({launches} launches)")
    return {"tok_s": B * steps / wall, "ms_per_token": ms, "launches_per_token": launches,
            "weight_copies_rotated": copies}


def bench_decode(args, dev):
    from swiftrwkv_amd import synthetic as syn

    model = DecodeModel(syn.X070_0B1, args.copies, dev, nthreads=min(16, os.cpu_count() or 1))
    step, wall, gpu_ms = run_decode(model, dev, 1, args.steps, args.warmup, args.copies)
    log(f"decode 0.1B: {args.steps} tokens, wall {wall * 1e3:.2f} ms, gpu {gpu_ms:.2f} ms")
    return model, step, wall, gpu_ms


def bench_decode_gemv(model, step, dev, reps=100):
    """Average in-graph duration of the GEMV kernel over the GEMV launches of
    a decode token: one HIP graph per weight copy holding only the token's
    GEMV launches (back to back, as in the token's graph), replayed over the
    rotated copies; per launch = replay time / launches.  Also returns the
    algorithmic bytes per launch (the token's packed weights + x + y over its
    GEMV launches)."""
    import torch

    copies = len(model.dev)
    n_gemv = model.launches_per_token
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        graphs = []
        for c in range(copies):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                step.launch(c, torch.cuda.current_stream().cuda_stream, gemv_only=True)
            graphs.append(g)
        for i in range(2 * copies):
            graphs[i % copies].replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(reps):
            graphs[i % copies].replay()
        e1.record(stream)
        torch.cuda.synchronize()
    return model.bytes_per_token / n_gemv, e0.elapsed_time(e1) / (reps * n_gemv), n_gemv


def bench_projection_crossover(model, dev, key="blocks.0.ffn.key.weight", reps=20):
    """Parallel-pass projection of N input rows through one weight matrix
    (the 0.1B ffn key, 3072x768): the GEMV kernel on the packed codes (all N
    rows in one launch) against dequantise to fp16 + matmul (hipBLASLt), the
    two branches of the model's baseProj.  Weights rotate over the copies."""
    import torch
    from swiftrwkv_amd import quant as Q

    qblk, qsqm, ddm, OUT, IN = model.host[key]
    copies = len(model.dev)
    stream = torch.cuda.current_stream(dev)
    res, cross = {}, None
    for N in (1, 4, 16, 64, 256, 1024):
        x = torch.randn((N, IN), device=dev)

        def gemv(c):
            q = model.dev[c][key]
            return Q.rwkvq_sb6_gemv(x, q[0], q[1], q[2], OUT, IN, 0)

        def deq_mm(c):
            q = model.dev[c][key]
            W = Q.rwkvq_dequant_dense(q[0], q[1], q[2], OUT, IN, 8, 0, torch.float16)
            return torch.nn.functional.linear(x.to(torch.float16), W).float()

        row = {}
        for name, fn in (("gemv_us", gemv), ("dequant_matmul_us", deq_mm)):
            for c in range(copies):
                fn(c)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for i in range(reps):
                fn(i % copies)
            e1.record(stream)
            torch.cuda.synchronize()
            row[name] = e0.elapsed_time(e1) * 1e3 / reps
        res[N] = row
        if cross is None and row["dequant_matmul_us"] < row["gemv_us"]:
            cross = N
    return {"shape": f"{OUT}x{IN} sb6 4-bit", "rows": res, "first_rows_where_dequant_matmul_wins": cross}


def bench_wkv_decode_step(dev, reps=30):
    """The fused WKV-7 decode step + tail (rwkv_wkv7_step_tail) alone, against
    its state-traffic roofline: per (row, head) the 64x64 fp32 state is read
    and written (32 KB) plus the step vectors, the tail's inputs and the
    output (13 · 64 · 4 B).  Rotating over 4 state buffers so the state comes
    from HBM when it exceeds the MALL."""
    import torch
    from swiftrwkv_amd import _lib

    res = {}
    for name, B, H in (("0.1B_batch1", 1, 12), ("0.1B_batch32", 32, 12), ("7B_batch16", 16, 64)):
        nb = 4
        states = [torch.zeros((B, H, 64, 64), device=dev) for _ in range(nb)]
        vec = [torch.randn((B, H, 64), device=dev) * 0.1 for _ in range(7)]
        r, w, k, v, a, b, g = vec
        w = torch.sigmoid(w) * 0.5 + 0.5
        rk, lnw, lnb = (torch.randn(H * 64, device=dev) for _ in range(3))
        out = torch.empty((B, H * 64), device=dev)
        stream = torch.cuda.current_stream(dev)

        def launch(i):
            st = states[i % nb]
            _lib.call("rwkv_wkv7_step_tail", *[z.data_ptr() for z in (r, w, k, v, a, b)], st.data_ptr(),
                      st.data_ptr(), rk.data_ptr(), lnw.data_ptr(), lnb.data_ptr(), g.data_ptr(), None,
                      out.data_ptr(), B, H, float(64e-5), stream.cuda_stream)

        for i in range(nb):
            launch(i)
        torch.cuda.synchronize()
        us = sum(kernel_ms(lambda: launch(i), stream) for i in range(reps)) / reps * 1e3
        nbytes = B * H * (2 * 64 * 64 * 4 + 13 * 64 * 4)
        roof_us = nbytes / (HBM_PEAK_GBPS * 1e3)
        res[name] = {"B": B, "H": H, "us": us, "bytes": nbytes, "GBps": nbytes / (us * 1e3),
                     "state_traffic_roofline_us": roof_us, "roofline_frac": roof_us / us}
        del states
    torch.cuda.empty_cache()
    return res


def bench_wkv_prefill_7b(dev, reps=3):
    """WKV-7 forward of one layer of the 7B-class prefill: B1 T8192 H64 fp32."""
    import torch
    from swiftrwkv_amd import kernel as K, synthetic as syn

    T, H, L = 8192, 64, 32
    x = [torch.from_numpy(z).to(dev) for z in syn.wkv_inputs_config0(1, T, H, seed=4)]
    K.wkv7_sequence_forward(*x)
    torch.cuda.synchronize()
    ms = sum(kernel_ms(lambda: K.wkv7_sequence_forward(*x)) for _ in range(reps)) / reps
    nbytes = T * H * 64 * (6 * 4 + 4) + 2 * H * 64 * 64 * 4
    flops = T * H * 9 * 64 * 64
    roof_ms = max(nbytes / (HBM_PEAK_GBPS * 1e9), flops / (VALU_PEAK_TFLOPS * 1e12)) * 1e3
    del x
    torch.cuda.empty_cache()
    return {"ms_per_layer": ms, "prefill_tok_s_32_layers": T / (L * ms * 1e-3), "bytes_per_layer": nbytes,
            "flop_per_layer": flops, "roofline_ms": roof_ms, "roofline_frac": roof_ms / ms}


def bench_decode_more(model_01, dev):
    """Batched decode of the 0.1B shape (B = 8, 32) and one-token decode of
    the 1.5B shape (24 layers, n_embd 2048, FFN 8192, vocab 65536; 776 MB of
    packed weights > the MALL, so one weight copy streams from HBM)."""
    import torch
    from swiftrwkv_amd import synthetic as syn

    res = {"projection_crossover_0.1B_ffn_key": bench_projection_crossover(model_01, dev)}
    log(f"projection crossover: {res['projection_crossover_0.1B_ffn_key']}")
    res["x070_decode_e2e_0.1B_batch8"] = x070_line(model_01, dev, 50, 5, copies=len(model_01.dev), B=8)
    for B in (8, 32):
        _, wall, gpu_ms = run_decode(model_01, dev, B, 50, 5, len(model_01.dev))
        res[f"decode_0.1B_batch{B}"] = {"tok_s": B * 50 / wall, "ms_per_step": wall * 1e3 / 50}
        log(f"decode 0.1B batch {B}: {wall * 1e3 / 50:.3f} ms per step")
    nthreads = min(16, os.cpu_count() or 1)
    # 0.4B (24 layers, n_embd 1024, FFN 4096): 2 weight copies (> the MALL)
    model = DecodeModel(syn.X070_0B4, 2, dev, nthreads=nthreads)
    for B in (1, 8, 32):
        _, wall, gpu_ms = run_decode(model, dev, B, 30, 4, 2)
        res[f"decode_0.4B_batch{B}"] = {"tok_s": B * 30 / wall, "ms_per_step": wall * 1e3 / 30}
        log(f"decode 0.4B batch {B}: {wall * 1e3 / 30:.3f} ms per step")
    del model
    torch.cuda.empty_cache()
    # 7B class (32 layers, n_embd 4096, FFN 14336): 3.57 GB of packed weights
    # per token; every layer has its own device buffers holding layer 0's bytes
    model = DecodeModel(syn.X070_7B, 1, dev, nthreads=nthreads, share_layers=True)
    for B in (1, 16):
        steps = 20 if B == 1 else 10
        _, wall, gpu_ms = run_decode(model, dev, B, steps, 2, 1)
        ms = wall * 1e3 / steps
        res[f"decode_7B_batch{B}"] = {"tok_s": B * steps / wall, "ms_per_step": ms,
                                      "gemv_bytes_per_token": model.bytes_per_token,
                                      "effective_GBps": model.bytes_per_token / (ms * 1e-3) / 1e9}
        log(f"decode 7B batch {B}: {ms:.3f} ms per step")
    res["x070_decode_e2e_7B_batch1"] = x070_line(model, dev, 20, 2)
    del model
    torch.cuda.empty_cache()
    res["wkv7_prefill_7B_B1_T8192_H64_fp32"] = bench_wkv_prefill_7b(dev)
    from swiftrwkv_amd import synthetic as syn
    res["wkv7_prefill_7B_B1_T8192_H64_fp32_chunked"] = bench_wkv_chunked(dev, 1, 8192, 64, syn.wkv_inputs_train,
                                                                         reps=3)
    res["wkv7_decode_step_tail"] = bench_wkv_decode_step(dev)
    log(f"decode step+tail: {res['wkv7_decode_step_tail']}")
    log("7B prefill WKV done")
    return res


def bench_prefill(dev, seconds_cap=60.0):
    """The parallel prefill pass (X070Decoder.prefill_batch, fp16 base: the
    sb6 projections on the matrix-core GEMM) of 128-token prompts of uniform
    random ids at the 0.1B and 0.4B shapes, batch 1 / 8 / 32, eager and
    replayed from its HIP graph (prefill_batch(graph=True)), and the whole
    generate_batch workload at batch 8 (128-token prefill, then 256 greedy
    steps); the 7B-class T = 8192 prefill; and the GEMM alone at the largest
    projection of each (its MFMA roofline)."""
    import numpy as np
    import torch
    from swiftrwkv_amd import quant as Q, synthetic as syn
    from swiftrwkv_amd.x070 import X070Decoder

    res = {}
    rng = np.random.default_rng(5)

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / reps

    def gemm_line(model, key, M):
        qblk, qsqm, ddm, OUT, IN = model.host[key]
        q = model.dev[0][key] if key in model.dev[0] else None
        if q is None:
            return None
        x = torch.randn((M, IN), device=dev).to(torch.float16)
        fl = 2 * M * OUT * IN
        # the long pass as the prefill calls it (with a workspace: the dequant
        # plus the dense kernel where the shape takes that route)
        ms = timed(lambda: Q.rwkvq_sb6_gemm(x, q[0], q[1], q[2], OUT, IN), 10) * 1e3
        tf = fl / (ms * 1e-3) / 1e12
        line = {"shape": f"{M}x{OUT}x{IN}", "ms": ms, "TFLOPs": tf, "mfma_fp16_peak_frac": tf / 2500.0,
                "route": "dequant + dense" if Q.rwkvq_gemm_workspace(M, OUT, IN) == OUT * IN * 2 else "fused"}
        # the fused kernel alone (no workspace) and the dense kernel alone
        ms_f = timed(lambda: Q.rwkvq_sb6_gemm(x, q[0], q[1], q[2], OUT, IN, split=False), 10) * 1e3
        line["fused_ms"], line["fused_peak_frac"] = ms_f, fl / (ms_f * 1e-3) / 1e12 / 2500.0
        if Q.rwkvq_f16_gemm_applies(M, OUT, IN):
            W = Q.rwkvq_dequant_dense(q[0], q[1], q[2], OUT, IN, 8, 0, torch.float16)
            ms_d = timed(lambda: Q.rwkvq_f16_gemm(x, W), 10) * 1e3
            line["dense_kernel_ms"], line["dense_peak_frac"] = ms_d, fl / (ms_d * 1e-3) / 1e12 / 2500.0
            del W
        return line

    nthreads = min(16, os.cpu_count() or 1)
    for shape in (syn.X070_0B1, syn.X070_0B4):
        model = DecodeModel(shape, 1, dev, nthreads=nthreads, share_layers=shape is syn.X070_0B4)
        dense = syn.x070_dense_params(shape, seed=11)
        dec = X070Decoder(shape.n_layer, shape.n_embd, shape.ffn, shape.vocab, dense, model.host, dev)
        for B in (1, 8, 32):
            prompts = [list(rng.integers(0, shape.vocab, 128)) for _ in range(B)]
            sec = timed(lambda: dec.prefill_batch(prompts, base_dtype=torch.float16), 3)
            # the same pass replayed from its HIP graph (captured in the untimed first call)
            sec_g = timed(lambda: dec.prefill_batch(prompts, base_dtype=torch.float16, graph=True), 5)
            res[f"prefill_{shape.name}_B{B}_T128_fp16base"] = {"ms": sec * 1e3, "tok_s": B * 128 / sec,
                                                              "ms_graph": sec_g * 1e3, "tok_s_graph": B * 128 / sec_g}
            log(f"prefill {shape.name} B{B} T128: {sec * 1e3:.2f} ms ({B * 128 / sec:.0f} tok/s), "
                f"graph {sec_g * 1e3:.2f} ms")
        prompts = [list(rng.integers(0, shape.vocab, 128)) for _ in range(8)]
        dec.generate_batch(prompts, 2)   # untimed: the batch's buffers and T16 weight copies are made here
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = dec.generate_batch(prompts, 256)
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
        res[f"generate_batch_{shape.name}_B8_prefill128_new256"] = {
            "s": el, "new_tok_s": sum(len(o) for o in out) / el,
            "note": "eager decode steps (no HIP graph), greedy choice on the host after each step"}
        log(f"generate_batch {shape.name} B8: {el:.2f} s")
        res[f"gemm_{shape.name}_ffn_key_M4096"] = gemm_line(model, "blocks.0.ffn.key.weight", 4096)
        del dec, model
        torch.cuda.empty_cache()
    # 7B class: one pass over a T = 8192 prompt, 32 layers sharing packed bytes
    shape = syn.X070_7B
    model = DecodeModel(shape, 1, dev, nthreads=nthreads, share_layers=True)
    dense = syn.x070_dense_params(shape, seed=11)
    dec = X070Decoder(shape.n_layer, shape.n_embd, shape.ffn, shape.vocab, dense, model.host, dev)
    prompt = [list(rng.integers(0, shape.vocab, 8192))]
    sec = timed(lambda: dec.prefill_batch(prompt, base_dtype=torch.float16), 3)
    res["prefill_7B_B1_T8192_fp16base"] = {"ms": sec * 1e3, "tok_s": 8192 / sec, "reps": 3}
    log(f"prefill 7B T8192: {sec * 1e3:.1f} ms")
    # batch 16 (the batched decode's prompts): 131,072 rows in one pass, ~61 GB of pass buffers
    prompts16 = [list(rng.integers(0, shape.vocab, 8192)) for _ in range(16)]
    sec16 = timed(lambda: dec.prefill_batch(prompts16, base_dtype=torch.float16), 1)
    res["prefill_7B_B16_T8192_fp16base"] = {"ms": sec16 * 1e3, "tok_s": 16 * 8192 / sec16, "reps": 1}
    log(f"prefill 7B B16 T8192: {sec16 * 1e3:.1f} ms")
    dec._tmp.clear()
    torch.cuda.empty_cache()
    res["gemm_7B_ffn_key_M8192"] = gemm_line(model, "blocks.0.ffn.key.weight", 8192)
    del dec, model
    torch.cuda.empty_cache()
    return res


def profile_prefill(dev):
    """Two passes of the 7B-class prefill over one 8192-token prompt (fp16
    base, 32 layers sharing packed bytes): the first makes the pass's buffers,
    the second is the one to read in a kernel trace."""
    import numpy as np
    import torch
    from swiftrwkv_amd import synthetic as syn
    from swiftrwkv_amd.x070 import X070Decoder

    shape = syn.X070_7B
    model = DecodeModel(shape, 1, dev, nthreads=min(16, os.cpu_count() or 1), share_layers=True)
    dense = syn.x070_dense_params(shape, seed=11)
    dec = X070Decoder(shape.n_layer, shape.n_embd, shape.ffn, shape.vocab, dense, model.host, dev)
    prompt = [list(np.random.default_rng(0).integers(0, shape.vocab, 8192))]
    for i in range(2):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dec.prefill_batch(prompt, base_dtype=torch.float16)
        torch.cuda.synchronize()
        log(f"prefill 7B T8192 pass {i}: {(time.perf_counter() - t0) * 1e3:.1f} ms")


def profile_prefill_short(dev):
    """The 0.1B prefill of one 128-token prompt (fp16 base): two eager passes
    (the first makes the buffers), then 20 replays of the pass's HIP graph,
    the ones to read in a kernel trace."""
    import numpy as np
    import torch
    from swiftrwkv_amd import synthetic as syn
    from swiftrwkv_amd.x070 import X070Decoder

    shape = syn.X070_0B1
    model = DecodeModel(shape, 1, dev, nthreads=min(16, os.cpu_count() or 1))
    dense = syn.x070_dense_params(shape, seed=11)
    dec = X070Decoder(shape.n_layer, shape.n_embd, shape.ffn, shape.vocab, dense, model.host, dev)
    prompt = [list(np.random.default_rng(5).integers(0, shape.vocab, 128))]
    for i in range(2):
        dec.prefill_batch(prompt, base_dtype=torch.float16)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(20):
        dec.prefill_batch(prompt, base_dtype=torch.float16, graph=True)
    torch.cuda.synchronize()
    log(f"prefill 0.1B B1 T128: {(time.perf_counter() - t0) / 20 * 1e3:.3f} ms per graph replay (with the first capture)")


def bench_head_gemv(model, dev, reps=60):
    """Average duration of the head GEMV over rotated weight copies (HBM)."""
    import torch
    from swiftrwkv_amd import _lib

    key = "head.weight"
    qblk, qsqm, ddm, OUT, IN = model.host[key]
    x = torch.randn((1, IN), device=dev)
    y = torch.empty((1, OUT), device=dev)
    L = _lib.lib()
    stream = torch.cuda.current_stream(dev)
    copies = len(model.dev)

    def launch(c):
        q = model.dev[c][key]
        _lib.check(L.rwkv_sb6_gemv(x.data_ptr(), 1, q[0].data_ptr(), q[1].data_ptr(), q[2].data_ptr(), y.data_ptr(),
                                   OUT, IN, 0, stream.cuda_stream))

    for i in range(10):
        launch(i % copies)
    torch.cuda.synchronize()
    durs = sorted(kernel_ms(lambda: launch(i % copies), stream) for i in range(reps))
    avg_ms = sum(durs) / len(durs)
    nbytes = qblk.nbytes + qsqm.nbytes + ddm.nbytes + 4 * (IN + OUT)
    return nbytes, avg_ms, durs[len(durs) // 2]


def bench_sym_gemv(dev, reps=60):
    """The sym GEMV (rwkv_sym_gemv, batch 1) on the 1.5B FFN shapes, 8- and
    6-bit: the average duration per launch (its own timestamps) over weight
    copies rotated through more than the 256 MB MALL, so every launch streams
    its matrix from HBM.  Bytes per launch = codes + group scales + super-block
    scales + the fp32 input and output rows.  The codes are random bytes and
    the scales small fp16 values (the kernel's work does not depend on them)."""
    import torch
    from swiftrwkv_amd import _lib

    L = _lib.lib()
    stream = torch.cuda.current_stream(dev)
    res = {}
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    for OUT, IN in ((8192, 2048), (2048, 8192)):
        for bits in (8, 6):
            NB = IN // 16
            qbytes = OUT * (IN if bits == 8 else IN // 32 * 24)
            per_copy = qbytes + OUT * NB + OUT * ((NB + 15) // 16) * 2
            copies = max(2, -(-300_000_000 // per_copy))
            bufs = []
            for _ in range(copies):
                q = torch.randint(0, 256, (qbytes,), dtype=torch.uint8, device=dev, generator=g)
                qs = torch.randint(0, 256, (OUT * NB,), dtype=torch.uint8, device=dev, generator=g)
                d = (torch.rand(OUT * ((NB + 15) // 16), device=dev, generator=g) * 1e-3).to(torch.float16)
                bufs.append((q, qs, d))
            x = torch.randn((1, IN), device=dev, generator=g)
            y = torch.empty((1, OUT), device=dev)

            def launch(c):
                q, qs, d = bufs[c % copies]
                _lib.check(L.rwkv_sym_gemv(x.data_ptr(), 1, q.data_ptr(), qs.data_ptr(), d.data_ptr(), y.data_ptr(),
                                           OUT, IN, bits, OUT, stream.cuda_stream))

            for i in range(2 * copies):
                launch(i)
            torch.cuda.synchronize()
            durs = [kernel_ms(lambda i=i: launch(i), stream) for i in range(reps)]
            avg_ms = sum(durs) / len(durs)
            nbytes = per_copy + 4 * (IN + OUT)
            gbps = nbytes / (avg_ms * 1e-3) / 1e9
            res[f"sym{bits}_gemv_{OUT}x{IN}"] = {"bytes": nbytes, "avg_us": avg_ms * 1e3, "GBps": gbps,
                                                 "hbm_frac": gbps / HBM_PEAK_GBPS, "weight_copies_rotated": copies}
            log(f"sym{bits} GEMV {OUT}x{IN}: {nbytes / 1e6:.2f} MB, avg {avg_ms * 1e3:.2f} us -> {gbps:.0f} GB/s")
            del bufs
            torch.cuda.empty_cache()
    return res


def bench_wkv(dev, reps=5):
    import numpy as np
    import torch
    from swiftrwkv_amd import kernel as K, synthetic as syn

    res = {}
    # config 0: B1 T1024 H12 fp32 forward
    x = [torch.from_numpy(z).to(dev) for z in syn.wkv_inputs_config0(1, 1024, 12, seed=0)]
    for _ in range(3):
        K.wkv7_sequence_forward(*x)
    torch.cuda.synchronize()
    ms = sum(kernel_ms(lambda: K.wkv7_sequence_forward(*x)) for _ in range(reps * 4)) / (reps * 4)
    nbytes = 1024 * 12 * 64 * 7 * 4 + 2 * 12 * 64 * 64 * 4
    res["wkv7_fwd_B1_T1024_H12_fp32"] = {"ms": ms, "tok_s": 1024 / (ms * 1e-3),
                                         "valu_roofline_frac": (1024 * 12 * 9 * 64 * 64 / (ms * 1e-3)) / (VALU_PEAK_TFLOPS * 1e12),
                                         "hbm_roofline_frac": nbytes / (ms * 1e-3) / (HBM_PEAK_GBPS * 1e9)}
    del x
    res["wkv7_fwd_B1_T1024_H12_fp32_chunked"] = bench_wkv_chunked(dev, 1, 1024, 12, syn.wkv_inputs_config0)
    # config 3: B8 T4096 H32 bf16 training forward (checkpointed) + backward
    B, T, H = 8, 4096, 32
    rng = np.random.default_rng(3)
    xs = syn.wkv_inputs_config0(B, T, H, seed=3)
    ins = [torch.from_numpy(z).to(dev).to(torch.bfloat16) for z in xs]
    del xs
    dy = torch.from_numpy(rng.standard_normal((B, T, H, 64), dtype=np.float32)).to(dev)
    ins_p, dt = K._prep(ins)
    grads = [torch.empty((B, T, H, 64), dtype=torch.bfloat16, device=dev) for _ in range(6)]
    dh_in = torch.empty((B, H, 64, 64), device=dev)
    from swiftrwkv_amd import _lib

    def fwd():
        return K._train_forward(ins_p, dt, None)

    def bwd(sa, ck):
        _lib.call("rwkv_wkv7_train_bwd", *[z.data_ptr() for z in ins_p], dt, None, ck.data_ptr(), sa.data_ptr(),
                  dy.data_ptr(), None, *[g.data_ptr() for g in grads], _lib.BF16, dh_in.data_ptr(), B, T, H, 2,
                  torch.cuda.current_stream().cuda_stream)

    out, h_out, sa, ck = fwd()
    bwd(sa, ck)
    torch.cuda.synchronize()
    tf = tb = 0.0
    res_fwd = {}
    for _ in range(reps):
        tf += kernel_ms(lambda: res_fwd.update(o=fwd()))
        out, h_out, sa, ck = res_fwd["o"]
        tb += kernel_ms(lambda: bwd(sa, ck))
    tf /= reps
    tb /= reps
    th = B * T * H
    res["wkv7_B8_T4096_H32_bf16"] = {
        "fwd_ms": tf, "bwd_ms": tb, "fwd_tok_s": B * T / (tf * 1e-3), "fwdbwd_tok_s": B * T / ((tf + tb) * 1e-3),
        "fwd_valu_roofline_frac": th * 9 * 4096 / (tf * 1e-3) / (VALU_PEAK_TFLOPS * 1e12),
        "bwd_valu_roofline_frac": th * 24 * 4096 / (tb * 1e-3) / (VALU_PEAK_TFLOPS * 1e12)}
    return res


def cpu_threads() -> int:
    """Threads for the CPU restatement: the host cores this process may run
    on, capped at the CPU share of one GPU (16) on an 8-GPU host."""
    from oracle import oracle as orc
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return max(1, min(16, avail, orc.max_threads()))


def cpu_baseline(model, step, seconds, dev):
    """The oracle's restatement of the non-kernel decode path on the host:
    every projection of one token dequantised to fp32 and multiplied in fp32
    (OpenMP over output rows), plus the MLX-op WKV step of every layer.  The
    CPU head output is first checked against the GPU head GEMV on the same
    packed bytes and input."""
    import numpy as np
    import torch
    from oracle import oracle as orc
    from swiftrwkv_amd import quant as Q

    nthreads = cpu_threads()
    xD = step.xD.cpu().numpy()[0]
    xF = step.xF.cpu().numpy()[0]
    xrkv = step.xrkv.cpu().numpy()
    vecs = [z.cpu().numpy() for z in step.rwkvab]
    state = np.zeros((step.L, 1, step.H, 64, 64), np.float32)
    out = np.empty((1, step.H, 64), np.float32)
    rkv_row = {"receptance": 0, "key": 1, "value": 2}
    ys = {}

    def token():
        for key, (qblk, qsqm, ddm, OUT, IN) in model.host.items():
            part = key.split(".")
            x = (xF if IN == step.F else
                 xrkv[rkv_row[part[3]]] if len(part) > 3 and part[2] == "att" and part[3] in rkv_row else xD)
            ys[key] = orc.cpu_sb6_dequant_matvec(x, qblk, qsqm, ddm, OUT, IN, 0, nthreads)
        for l in range(step.L):
            r, w, k, v, a, b = (np.ascontiguousarray(z[l]) for z in vecs)
            orc.cpu_wkv7_step(r, w, k, v, a, b, state[l], out, 1, step.H, nthreads)

    t0 = time.perf_counter()
    token()
    first = time.perf_counter() - t0
    # the CPU head equals the GPU head GEMV (same bytes, same x) within the GEMV tolerance
    q = model.dev[0]["head.weight"]
    OUT, IN = model.host["head.weight"][3:5]
    gpu = Q.rwkvq_sb6_gemv(step.xD, q[0], q[1], q[2], OUT, IN, 0)[0].cpu().numpy().astype(np.float64)
    err = float(np.abs(gpu - ys["head.weight"]).max() / np.abs(gpu).max())
    if not err < 1e-5:
        raise RuntimeError(f"CPU head differs from the GPU head GEMV: rel {err:.3e}")
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds and n < 2000:
        token()
        n += 1
    el = time.perf_counter() - t0
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {"value": n / el, "unit": "tok/s", "cores": nthreads, "kind": "port",
            "sample": f"{n} decode tokens of the {model.shape.name} shape ({len(model.host)} sb6 dequant+fp32 "
                      f"matvecs + {step.L} WKV steps each; first token {first:.2f} s), {el:.1f} s on {nthreads} "
                      f"OpenMP threads ({avail} cores visible); CPU head vs GPU head GEMV rel {err:.1e}"}


def cpu_wkv_baseline():
    import numpy as np
    from oracle import oracle as orc
    from swiftrwkv_amd import synthetic as syn

    x = syn.wkv_inputs_config0(1, 1024, 12, seed=0)
    nthreads = cpu_threads()
    orc.wkv7_fwd_f32(*x, nthreads=nthreads)
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < 2.0:
        orc.wkv7_fwd_f32(*x, nthreads=nthreads)
        n += 1
    el = (time.perf_counter() - t0) / n
    return {"value": 1024 / el, "unit": "tok/s", "cores": nthreads, "kind": "port",
            "sample": f"WKV-7 forward B1 T1024 H12 fp32 x{n}"}


def profile_kernels(dev, tokens=12):
    """The dominant kernels alone, for rocprofv3: eager 0.1B decode tokens over
    6 rotated weight copies (49 GEMV launches each, the head GEMV among them,
    and 12 WKV step+tail launches), 6 eager 1.5B decode tokens (97 GEMV
    launches each), 4 eager tokens of the whole 1.5B x070 step (123 launches
    each), the WKV-7 forward at B1 T1024 H12 fp32 (20 launches), the
    time-chunked forward at B1 T1024 H12 (5) and B1 T8192 H64 (2), the
    batched GEMV of a 14336x4096 matrix x 16 rows on the matrix cores over
    K3 weights, over T16 weights and on the VALU kernel (3 each), the
    checkpointed training forward +
    backward at B8 T4096 H32 bf16 (3 each),
    and a plain 256 MiB device copy whose FETCH_SIZE / WRITE_SIZE calibrate
    the counters (2 x 256 MiB of traffic)."""
    import numpy as np
    import torch
    from swiftrwkv_amd import _lib, kernel as K, synthetic as syn

    src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    model = DecodeModel(syn.X070_0B1, 6, dev, nthreads=min(16, os.cpu_count() or 1))
    step = DecodeStep(model, dev, B=1)
    stream = torch.cuda.current_stream(dev).cuda_stream
    for i in range(tokens):
        step.launch(i % 6, stream)
    torch.cuda.synchronize()
    log("decode tokens done")
    del model, step
    model = DecodeModel(syn.X070_1B5, 1, dev, nthreads=min(16, os.cpu_count() or 1))
    step = DecodeStep(model, dev, B=1)
    for _ in range(6):
        step.launch(0, stream)
    torch.cuda.synchronize()
    del step
    log("1.5B decode tokens done")
    # 4 eager tokens of the whole 1.5B x070 step (the headline's kernels:
    # rkv_lora_ln, tmix_core, o_proj, gemv_ln, ffn value per layer, the head)
    from swiftrwkv_amd.x070 import X070Decoder
    s = syn.X070_1B5
    dec = X070Decoder(s.n_layer, s.n_embd, s.ffn, s.vocab, syn.x070_dense_params(s, seed=11), model.host, dev)
    st = dec.new_state(1)
    ids = torch.randint(0, s.vocab, (1,), dtype=torch.int32, device=dev)
    for _ in range(4):
        dec.launch(ids, st)
    torch.cuda.synchronize()
    del model, dec, st
    torch.cuda.empty_cache()
    log("1.5B x070 step tokens done")
    x = [torch.from_numpy(z).to(dev) for z in syn.wkv_inputs_config0(1, 1024, 12, seed=0)]
    for _ in range(20):
        K.wkv7_sequence_forward(*x)
    for _ in range(5):
        K.wkv7_sequence_forward_chunked(*x)
    x7 = [torch.from_numpy(z).to(dev) for z in syn.wkv_inputs_train(1, 8192, 64, seed=0)]
    for _ in range(2):
        K.wkv7_sequence_forward_chunked(*x7)
    del x7
    # batched decode GEMV, 7B-class FFN key 14336x4096 x 16 rows: matrix cores, then the VALU kernel
    from swiftrwkv_amd import quant as Q
    OUT, IN, N = 14336, 4096, 16
    w = np.random.default_rng(3).standard_normal((OUT, IN), dtype=np.float32) * np.float32(0.02)
    disk = Q.encode_sb6(w, 4, min(16, os.cpu_count() or 1))
    qb, qs, dd, _ = Q.rwkvq_sb6_to_k3(disk["codes_packed"], disk["gw_qsqm"], disk["gw_d"], disk["gw_dm"], None,
                                      None, (OUT, IN))
    qb, qs, dd = (torch.from_numpy(z).to(dev) for z in (qb, qs, dd.view(np.float16)))
    xb = torch.randn((N, IN), device=dev)
    for _ in range(3):
        Q.rwkvq_sb6_gemv_batch(xb, qb, qs, dd, OUT, IN)
    t16 = Q.rwkvq_sb6_t16(qb, qs, dd, OUT, IN)
    for _ in range(3):
        Q.rwkvq_sb6_gemv_batch_t16(xb, *t16, OUT, IN)
    for _ in range(3):
        Q.rwkvq_sb6_gemv(xb, qb, qs, dd, OUT, IN, 0)
    del qb, qs, dd, xb, t16
    B, T, H = 8, 4096, 32
    xs = syn.wkv_inputs_config0(B, T, H, seed=3)
    ins = [torch.from_numpy(z).to(dev).to(torch.bfloat16) for z in xs]
    ins_p, dt = K._prep(ins)
    dy = torch.randn((B, T, H, 64), device=dev)
    grads = [torch.empty((B, T, H, 64), dtype=torch.bfloat16, device=dev) for _ in range(6)]
    dh_in = torch.empty((B, H, 64, 64), device=dev)
    for _ in range(3):
        out, h_out, sa, ck = K._train_forward(ins_p, dt, None)
        _lib.call("rwkv_wkv7_train_bwd", *[z.data_ptr() for z in ins_p], dt, None, ck.data_ptr(), sa.data_ptr(),
                  dy.data_ptr(), None, *[g.data_ptr() for g in grads], _lib.BF16, dh_in.data_ptr(), B, T, H, 2,
                  torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    log("kernels done")


def profile_step(dev, tokens=4, replays=20):
    """The 1.5B headline step alone, for rocprofv3 counter passes: a plain
    256 MiB device copy (the counters' calibration), `tokens` eager x070
    decode tokens of the 1.5B shape (123 launches each: per layer
    rkv_lora_ln, tmix_core, o_proj, gemv_ln, ffn value; emb + ln0, ln_out,
    head), then `replays` replays of the token's HIP graph, then 5 + `replays`
    replays of the graph the headline's roofline is measured on (the same
    step without its tmix cores and layer norms)."""
    import torch
    from swiftrwkv_amd import synthetic as syn
    from swiftrwkv_amd.x070 import X070Decoder

    src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    s = syn.X070_1B5
    model = DecodeModel(s, 1, dev, nthreads=min(16, os.cpu_count() or 1))
    dec = X070Decoder(s.n_layer, s.n_embd, s.ffn, s.vocab, syn.x070_dense_params(s, seed=11), model.host, dev)
    st = dec.new_state(1)
    ids = torch.randint(0, s.vocab, (1,), dtype=torch.int32, device=dev)
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        for _ in range(tokens):
            dec.launch(ids, st)
        torch.cuda.synchronize()
        log("eager tokens done")
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            dec.launch(ids, st)
        for _ in range(replays):
            g.replay()
        torch.cuda.synchronize()
    log("graph replays done")
    del dec, st, g
    torch.cuda.empty_cache()
    # the roofline's graph: the same step without its tmix cores and layer norms
    _, n, avg_ms, _ = bench_step_gemv_launches(model, dev, reps=replays)
    log(f"GEMV-bearing launches graph: {n} launches, {avg_ms * 1e3:.2f} us per launch")


def profile_x070(dev, tokens=20):
    """End-to-end x070 decode tokens (HIP graph replays) of the 0.1B and
    7B-class shapes, batch 1, for kernel traces."""
    import torch
    from swiftrwkv_amd import synthetic as syn

    nthreads = min(16, os.cpu_count() or 1)
    for shape in (syn.X070_0B1, syn.X070_7B):
        model = DecodeModel(shape, 1, dev, nthreads=nthreads, share_layers=shape is syn.X070_7B)
        wall, _, launches = run_x070(model, dev, tokens, 2)
        log(f"x070 decode {shape.name}: {wall * 1e3 / tokens:.3f} ms per token, {launches} launches")
        del model
        torch.cuda.empty_cache()


def profile_batch(dev, steps=20):
    """Batched decode steps (GEMV + WKV chain, HIP graph replays) of the 0.1B
    (batch 8, 32), 0.4B (8, 32) and 7B-class (16) shapes, for kernel traces;
    the shapes run in that order."""
    import torch
    from swiftrwkv_amd import synthetic as syn

    nthreads = min(16, os.cpu_count() or 1)
    for shape, copies, batches in ((syn.X070_0B1, 6, (8, 32)), (syn.X070_0B4, 2, (8, 32)), (syn.X070_7B, 1, (16,))):
        model = DecodeModel(shape, copies, dev, nthreads=nthreads, share_layers=shape is syn.X070_7B)
        for B in batches:
            _, wall, _ = run_decode(model, dev, B, steps, 2, copies)
            log(f"batched decode {shape.name} batch {B}: {wall * 1e3 / steps:.3f} ms per step")
        del model
        torch.cuda.empty_cache()


def headline_1b5(args, dev):
    """The 1.5B decode: the whole x070 step per token (the headline), the
    GEMV + WKV chain of the same token, the GEMV roofline and the CPU baseline."""
    from swiftrwkv_amd import synthetic as syn

    model = DecodeModel(syn.X070_1B5, 1, dev, nthreads=min(16, os.cpu_count() or 1))
    wall, gpu_ms, launches = run_x070(model, dev, args.steps, args.warmup)
    log(f"x070 decode 1.5B: {args.steps} tokens, wall {wall * 1e3:.2f} ms, gpu {gpu_ms:.2f} ms, {launches} launches")
    # the roofline: the timed step's own GEMV-bearing launches, in step order
    sb_bytes, n_sb, sb_avg_ms, token_bytes = bench_step_gemv_launches(model, dev)
    achieved = sb_bytes / (n_sb * sb_avg_ms * 1e-3) / 1e9
    log(f"1.5B step GEMV-bearing launches: {n_sb} per token, {sb_bytes / 1e6:.1f} MB, avg {sb_avg_ms * 1e3:.2f} us "
        f"-> {achieved:.0f} GB/s; whole token {token_bytes / 1e6:.1f} MB")
    step, cwall, cgpu = run_decode(model, dev, 1, 100, 10, 1)
    gemv_bytes, gemv_avg_ms, n_gemv = bench_decode_gemv(model, step, dev)
    gemv_only = gemv_bytes / (gemv_avg_ms * 1e-3) / 1e9
    log(f"1.5B decode GEMV (plain launches): {n_gemv} launches per token, {gemv_bytes / 1e6:.3f} MB per launch, "
        f"avg {gemv_avg_ms * 1e3:.2f} us -> {gemv_only:.0f} GB/s")
    chain = {"tok_s": 100 / cwall, "ms_per_token": cwall * 10, "gemv_bytes_per_token": model.bytes_per_token,
             "effective_GBps": model.bytes_per_token / (cwall * 1e-2) / 1e9,
             "gemv_launches_per_token": n_gemv, "gemv_avg_us": gemv_avg_ms * 1e3,
             "gemv_kernel_us_per_token": gemv_avg_ms * 1e3 * n_gemv,
             "gemv_hbm_frac": gemv_only / HBM_PEAK_GBPS, "gemv_traffic": DECODE_1B5_GEMV_TRAFFIC_BYTES}
    cpu = None if args.skip_cpu else cpu_baseline(model, step, args.cpu_seconds, dev)
    # the same chain for 16 rows (batched decode: the matrix-core GEMVs over T16 copies)
    del step
    _, bwall, _ = run_decode(model, dev, 16, 30, 4, 1)
    batch16 = {"tok_s": 16 * 30 / bwall, "ms_per_step": bwall * 1e3 / 30}
    log(f"1.5B decode batch 16: {bwall * 1e3 / 30:.3f} ms per step")
    res = {"wall": wall, "gpu_ms": gpu_ms, "launches": launches, "achieved": achieved, "n_sb": n_sb,
           "sb_bytes": sb_bytes, "sb_avg_ms": sb_avg_ms, "token_bytes": token_bytes, "chain": chain, "cpu": cpu,
           "batch16": batch16}
    del model
    import torch
    torch.cuda.empty_cache()
    return res


def config1_0b1(args, dev):
    """One-token decode of the 0.1B shape: the GEMV + WKV chain (73 GEMVs as
    49 launches and 12 step+tail launches, rotated weight copies), its GEMV
    roofline, the head GEMV alone, the whole step, and the CPU baseline."""
    model, step, wall, gpu_ms = bench_decode(args, dev)
    gemv_bytes, gemv_avg_ms, n_gemv = bench_decode_gemv(model, step, dev)
    achieved = gemv_bytes / (gemv_avg_ms * 1e-3) / 1e9
    log(f"0.1B decode GEMV: {n_gemv} launches per token, {gemv_bytes / 1e6:.3f} MB per launch, "
        f"avg {gemv_avg_ms * 1e3:.2f} us -> {achieved:.0f} GB/s")
    nbytes, head_avg_ms, head_med_ms = bench_head_gemv(model, dev)
    head_gbps = nbytes / (head_avg_ms * 1e-3) / 1e9
    log(f"head GEMV: {nbytes / 1e6:.2f} MB, avg {head_avg_ms * 1e3:.1f} us -> {head_gbps:.0f} GB/s")
    steps = args.steps
    res = {
        "decode_0.1B_gemv_wkv_chain_batch1": {
            "tok_s": steps / wall, "ms_per_token": wall * 1e3 / steps, "gpu_ms_per_token": gpu_ms / steps,
            "gemv_bytes_per_token": model.bytes_per_token,
            "effective_GBps": model.bytes_per_token / (gpu_ms * 1e-3 / steps) / 1e9,
            "launches_per_token": n_gemv + 12, "weight_copies_rotated": args.copies,
            "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": achieved / HBM_PEAK_GBPS, "traffic": DECODE_GEMV_TRAFFIC_BYTES,
                         "kernel": f"gemv_kernel, in-graph average over the {n_gemv} GEMV launches of one token"}},
        "head_gemv_65536x768": {"bytes": nbytes, "avg_us": head_avg_ms * 1e3, "median_us": head_med_ms * 1e3,
                                "GBps": head_gbps, "hbm_frac": head_gbps / HBM_PEAK_GBPS,
                                "traffic": HEAD_GEMV_TRAFFIC_BYTES},
        "x070_decode_e2e_0.1B_batch1": x070_line(model, dev, 200, 10, copies=len(model.dev)),
    }
    if not args.skip_cpu:
        res["decode_0.1B_gemv_wkv_chain_batch1"]["cpu_baseline"] = cpu_baseline(model, step, min(5.0, args.cpu_seconds),
                                                                                 dev)
    return model, res


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); "
              "the path runs on one GPU; how it would shard is described, not built", file=sys.stderr)
        sys.exit(1)
    import torch
    from swiftrwkv_amd import _lib

    _lib.lib()
    dev = torch.device("cuda:0")
    log(f"device {torch.cuda.get_device_name(0)}")
    if args.mode == "kernels":
        profile_kernels(dev)
        return
    if args.mode == "e2e":
        profile_x070(dev)
        return
    if args.mode == "batch":
        profile_batch(dev)
        return
    if args.mode == "step":
        profile_step(dev)
        return
    if args.mode == "prefill":
        profile_prefill(dev)
        return
    if args.mode == "prefill_short":
        profile_prefill_short(dev)
        return
    head = headline_1b5(args, dev)
    extra = {"decode_1.5B_gemv_wkv_chain_batch1": head["chain"], "decode_1.5B_batch16": head["batch16"]}
    model01, more01 = config1_0b1(args, dev)
    extra.update(more01)
    extra.update(bench_sym_gemv(dev))
    if not args.skip_wkv:
        extra.update(bench_wkv(dev))
        log("wkv done")
    if not args.skip_more:
        extra.update(bench_decode_more(model01, dev))
        extra.update(bench_prefill(dev))
    if not args.skip_cpu:
        extra["cpu_wkv7_fwd_B1_T1024_H12"] = cpu_wkv_baseline()
        log("cpu baseline done")
    wall = head["wall"]
    line = {
        "metric": METRIC, "value": args.steps / wall, "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": wall * 1e3 / args.steps, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "1.5B decode: one-token x070 decode step of the 1.5B shape, batch 1, end to end "
                               "(embedding row to logits) in one HIP graph: per layer ln1 + token shift + 6 "
                               "lerps, fused r/k/v sb6 GEMV with the low-rank first layers, tmix core (low-rank "
                               "second layers, WKV-7 step, group-norm tail, gate), o_proj + residual, ln2 + "
                               "shift, ffn key relu², ffn value + residual; ln_out, head",
                   "n_layer": 24, "n_embd": 2048, "n_head": 32, "ffn": 8192, "vocab": 65536, "batch": 1,
                   "weights": "sb6 4-bit from seeded N(0,0.02), 776 MB packed per token; dense parameters "
                              "seeded, low-rank matrices fp16",
                   "launches_per_token": head["launches"], "hip_graph_per_token": True},
        "roofline": {"bound": "hbm", "achieved": head["achieved"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": head["achieved"] / HBM_PEAK_GBPS, "traffic": DECODE_1B5_STEP_GEMV_TRAFFIC_BYTES,
                     "kernel": f"the timed step's own GEMV-bearing launches ({head['n_sb']} per token: per layer "
                               f"rkv_lora_ln_kernel, o_proj + residual gemv_kernel, gemv_ln_kernel (ffn key), "
                               f"ffn value + residual gemv_kernel; the head), replayed back to back in step order "
                               f"from a graph of the step without its tmix cores and layer norms; average "
                               f"{head['sb_avg_ms'] * 1e3:.2f} us per launch; bytes per launch = packed "
                               f"projections + fp16 low-rank inner matrices + fp32 rows / launches = "
                               f"{head['sb_bytes'] / head['n_sb']:.0f}",
                     "whole_token": {"bytes": head["token_bytes"],
                                     "achieved": head["token_bytes"] / (wall / args.steps) / 1e9,
                                     "frac": head["token_bytes"] / (wall / args.steps) / 1e9 / HBM_PEAK_GBPS}},
        "cpu_baseline": head["cpu"],
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
