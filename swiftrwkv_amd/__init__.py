"""swiftrwkv_amd — MI355X (gfx950) implementation of SwiftRWKV's data-parallel
hot path: the WKV-7 recurrence (RWKVKernel) and the .rwkvq dequant / decode
GEMV (RWKVQuant), behind a plain C ABI (include/rwkv_hip.h) with a Python
mirror of the reference's Swift API.

    swiftrwkv_amd.kernel     RWKVKernel API (wkv7_sequence_forward, wkv7_train_with_state, ...)
    swiftrwkv_amd.quant      RWKVQuant API (RwkvqSidecar, rwkvq_sb6_gemv, ...)
    swiftrwkv_amd.synthetic  seeded inputs / weights of the benchmark shapes
    swiftrwkv_amd.build      builds libswiftrwkv_hip.so in-tree
"""
from . import _lib  # noqa: F401

__all__ = ["kernel", "quant", "synthetic", "build"]
