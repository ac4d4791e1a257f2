"""The WKV-7 chunked forward that allocates nothing
(rwkv_wkv7_seq_fwd_chunked_static) against the workspace entry point
(rwkv_wkv7_seq_fwd_chunked) through the C ABI: the same kernels over the
library's static device scratch, so outputs and states are bitwise equal.
Two calls in a row, the second smaller, so stale scratch from the first
cannot leak into the second; sizes beyond the scratch are refused."""
import sys

import numpy as np
import pytest
import torch

from swiftrwkv_amd import _lib, kernel as K
from swiftrwkv_amd import synthetic as syn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def call_static(x, h0, B, T, H, dt=_lib.F32):
    out = torch.empty((B, T, H, 64), dtype=torch.float32, device=DEV)
    h = torch.empty((B, H, 64, 64), dtype=torch.float32, device=DEV)
    st = _lib.lib().rwkv_wkv7_seq_fwd_chunked_static(*[z.data_ptr() for z in x], dt,
                                                     None if h0 is None else h0.data_ptr(), out.data_ptr(),
                                                     h.data_ptr(), B, T, H,
                                                     torch.cuda.current_stream().cuda_stream)
    return st, out, h


def test_static_scratch_equals_workspace_entry():
    for (B, T, H, seed) in [(1, 1024, 12, 0), (2, 77, 3, 1)]:
        case(f"static-scratch chunked fwd B{B} T{T} H{H}")
        x = [torch.from_numpy(z).to(DEV) for z in syn.wkv_inputs_config0(B, T, H, seed=seed)]
        h0 = torch.from_numpy(syn.state(B, H, seed=seed)).to(DEV)
        want_o, want_h = K.wkv7_sequence_forward_chunked(*x, h_in=h0)
        st, out, h = call_static(x, h0, B, T, H)
        torch.cuda.synchronize()
        assert st == 0, _lib.lib().rwkv_last_error()
        assert torch.equal(out, want_o) and torch.equal(h, want_h)
        assert out.abs().sum() > 0


def test_static_scratch_refuses_passes_beyond_it():
    case("static-scratch chunked fwd: too large is refused before any launch")
    B, T, H = 1, 32, 1
    x = [torch.zeros((B, T, H, 64), device=DEV) for _ in range(6)]
    before = _lib.counters()["seq_chunked"]
    # 1366 chunk-heads: one more than the 64 MiB scratch holds
    st = _lib.lib().rwkv_wkv7_seq_fwd_chunked_static(*[z.data_ptr() for z in x], _lib.F32, None,
                                                     x[0].data_ptr(), x[1].data_ptr(), 1, 32 * 1366, 1, None)
    assert st != 0 and b"static scratch" in _lib.lib().rwkv_last_error()
    # sizes whose byte count would wrap a 64-bit product (T = 2^55 gives
    # 2^50 chunks: × 48 KiB is 0 mod 2^64) are refused as well
    for (b_, t_, h_) in [(1, 1 << 55, 1), (1 << 40, 32, 1 << 30), (1, (1 << 63) - 1, 1), (1366, 1, 1)]:
        st = _lib.lib().rwkv_wkv7_seq_fwd_chunked_static(*[z.data_ptr() for z in x], _lib.F32, None,
                                                         x[0].data_ptr(), x[1].data_ptr(), b_, t_, h_, None)
        assert st != 0 and b"static scratch" in _lib.lib().rwkv_last_error(), (b_, t_, h_)
    assert _lib.counters()["seq_chunked"] == before
