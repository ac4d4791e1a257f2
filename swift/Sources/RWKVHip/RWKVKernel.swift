// RWKVKernel over the MI355X C ABI: the public functions of
// Sources/RWKVKernel/WKV7.swift, WKV7Train.swift and WKV7DecodeKernels.swift
// with the reference's names, argument order and switches.  Where the
// reference traps (precondition) these throw RWKVHipError; shapes are
// [B, T, H, 64] for sequence inputs and [B, H, 64, 64] for states.

import CRwkvHip

public let WKV7_HEAD_SIZE = 64   // WKV7.swift:7
public let WKV7_CHUNK = 16       // WKV7.swift:8

/// WKV7.swift:178 — whole sequence in one launch (true) or 16-token chunks.
nonisolated(unsafe) public var wkv7WholeSequenceForward = true
/// WKV7Train.swift:343-354 — backward variant and keep-vs-recompute.
nonisolated(unsafe) public var wkv7BackwardV2 = true

/// WKV7.swift:181, WKV7Train.swift:358 — launch counters, from the library.
public var wkv7SequenceLaunches: Int { Int(counters().seq_fwd) }
public var wkv7TrainForwardLaunches: Int { Int(counters().train_fwd) }

func counters() -> rwkv_counters {
    var c = rwkv_counters()
    rwkv_get_counters(&c)
    return c
}

private func btph(_ r: DeviceArray) throws -> (Int, Int, Int) {
    guard r.shape.count == 4, r.shape[3] == WKV7_HEAD_SIZE else {
        throw RWKVHipError.status(Int32(RWKV_E_SHAPE.rawValue), "inputs must be [B, T, H, \(WKV7_HEAD_SIZE)], got \(r.shape)")
    }
    return (r.shape[0], r.shape[1], r.shape[2])
}

/// WKV7.swift:242-264 — the frozen forward over the whole sequence in one launch.
public func wkv7SequenceForward(_ r: DeviceArray, _ w: DeviceArray, _ k: DeviceArray, _ v: DeviceArray,
                                _ a: DeviceArray, _ b: DeviceArray, _ hIn: DeviceArray? = nil) throws
    -> (DeviceArray, DeviceArray) {
    let (B, T, H) = try btph(r)
    let out = try DeviceArray(shape: [B, T, H, WKV7_HEAD_SIZE], dtype: .float32)
    let hOut = try DeviceArray(shape: [B, H, WKV7_HEAD_SIZE, WKV7_HEAD_SIZE], dtype: .float32)
    try check(rwkv_wkv7_seq_fwd(r.raw, w.raw, k.raw, v.raw, a.raw, b.raw, r.dtype.code, hIn?.f32, out.f32, hOut.f32,
                                Int64(B), Int64(T), Int64(H), streamArg))
    return (out, hOut)
}

/// WKV7.swift:64-82 — one 16-token chunk, also returning sa = S·a per step.
public func wkv7ChunkForward(_ r: DeviceArray, _ w: DeviceArray, _ k: DeviceArray, _ v: DeviceArray,
                             _ a: DeviceArray, _ b: DeviceArray, _ hIn: DeviceArray) throws
    -> (DeviceArray, DeviceArray, DeviceArray) {
    let (B, T, H) = try btph(r)
    let out = try DeviceArray(shape: [B, T, H, WKV7_HEAD_SIZE], dtype: .float32)
    let hOut = try DeviceArray(shape: [B, H, WKV7_HEAD_SIZE, WKV7_HEAD_SIZE], dtype: .float32)
    let sa = try DeviceArray(shape: [B, T, H, WKV7_HEAD_SIZE], dtype: .float32)
    try check(rwkv_wkv7_chunk_fwd(r.raw, w.raw, k.raw, v.raw, a.raw, b.raw, r.dtype.code, hIn.f32, out.f32, hOut.f32,
                                  sa.f32, Int64(B), Int64(T), Int64(H), streamArg))
    return (out, hOut, sa)
}

/// WKV7.swift:96-103 — dispatch by `wkv7WholeSequenceForward`; both arms give
/// the same bits.
public func wkv7ForwardWithState(_ r: DeviceArray, _ w: DeviceArray, _ k: DeviceArray, _ v: DeviceArray,
                                 _ a: DeviceArray, _ b: DeviceArray, _ hIn: DeviceArray? = nil) throws
    -> (DeviceArray, DeviceArray) {
    if wkv7WholeSequenceForward { return try wkv7SequenceForward(r, w, k, v, a, b, hIn) }
    return try wkv7ForwardChunked(r, w, k, v, a, b, hIn)
}

/// WKV7.swift:107-140 — 16 tokens per launch (the tail padded with neutral
/// steps by the caller's T % 16 == 0 here; a ragged tail goes to the
/// whole-sequence launch, which gives the same bits).
public func wkv7ForwardChunked(_ r: DeviceArray, _ w: DeviceArray, _ k: DeviceArray, _ v: DeviceArray,
                               _ a: DeviceArray, _ b: DeviceArray, _ hIn: DeviceArray? = nil) throws
    -> (DeviceArray, DeviceArray) {
    let (B, T, H) = try btph(r)
    guard T % WKV7_CHUNK == 0 else { return try wkv7SequenceForward(r, w, k, v, a, b, hIn) }
    let D = WKV7_HEAD_SIZE
    var h = try hIn ?? DeviceArray.zeros([B, H, D, D])
    let out = try DeviceArray(shape: [B, T, H, D], dtype: .float32)
    // per chunk: the [B, 16, H, 64] slice of every input is a strided view in
    // [B, T, H, 64]; stage each into a contiguous chunk buffer
    let es = r.dtype.size
    let chunkIn = try (0 ..< 6).map { _ in try DeviceArray(shape: [B, WKV7_CHUNK, H, D], dtype: r.dtype) }
    let oc = try DeviceArray(shape: [B, WKV7_CHUNK, H, D], dtype: .float32)
    let sa = try DeviceArray(shape: [B, WKV7_CHUNK, H, D], dtype: .float32)
    let rowBytes = H * D * es
    for c in 0 ..< T / WKV7_CHUNK {
        for (src, dst) in zip([r, w, k, v, a, b], chunkIn) {
            guard hipMemcpy2DAsync(dst.raw, WKV7_CHUNK * rowBytes, src.raw + c * WKV7_CHUNK * rowBytes, T * rowBytes,
                                   WKV7_CHUNK * rowBytes, B, hipMemcpyDeviceToDevice, rwkvHipStream) == hipSuccess
            else { throw RWKVHipError.hip("hipMemcpy2DAsync failed") }
        }
        let hNext = try DeviceArray(shape: [B, H, D, D], dtype: .float32)
        try check(rwkv_wkv7_chunk_fwd(chunkIn[0].raw, chunkIn[1].raw, chunkIn[2].raw, chunkIn[3].raw, chunkIn[4].raw,
                                      chunkIn[5].raw, r.dtype.code, h.f32, oc.f32, hNext.f32, sa.f32, Int64(B),
                                      Int64(WKV7_CHUNK), Int64(H), streamArg))
        guard hipMemcpy2DAsync(out.raw + c * WKV7_CHUNK * H * D * 4, T * H * D * 4, oc.raw, WKV7_CHUNK * H * D * 4,
                               WKV7_CHUNK * H * D * 4, B, hipMemcpyDeviceToDevice, rwkvHipStream) == hipSuccess
        else { throw RWKVHipError.hip("hipMemcpy2DAsync failed") }
        h = hNext
    }
    return (out, h)
}

/// WKV7.swift:143-148 — zero initial state, final state dropped.
public func wkv7Forward(_ r: DeviceArray, _ w: DeviceArray, _ k: DeviceArray, _ v: DeviceArray,
                        _ a: DeviceArray, _ b: DeviceArray) throws -> DeviceArray {
    try wkv7ForwardWithState(r, w, k, v, a, b, nil).0
}

/// What the training forward keeps for its backward (WKV7Train.swift:390-397):
/// the per-step sa and the state after every 16-token chunk.
public struct WKV7TrainSaved {
    public let sa: DeviceArray       // [B, T, H, 64]
    public let hCkpt: DeviceArray    // [B, H, T/16, 64, 64]
    public let hIn: DeviceArray?
}

/// WKV7Train.swift:375-470, forward half: (out, h_out) and the tensors the
/// VJP needs.  Autograd stays in the caller (the reference's CustomFunction);
/// `wkv7TrainBackward` is its VJP body.  Requires T % 16 == 0.
public func wkv7TrainWithState(_ r: DeviceArray, _ w: DeviceArray, _ k: DeviceArray, _ v: DeviceArray,
                               _ a: DeviceArray, _ b: DeviceArray, _ hIn: DeviceArray? = nil) throws
    -> (DeviceArray, DeviceArray, WKV7TrainSaved) {
    let (B, T, H) = try btph(r)
    let D = WKV7_HEAD_SIZE
    let out = try DeviceArray(shape: [B, T, H, D], dtype: .float32)
    let hOut = try DeviceArray(shape: [B, H, D, D], dtype: .float32)
    let sa = try DeviceArray(shape: [B, T, H, D], dtype: .float32)
    let ck = try DeviceArray(shape: [B, H, max(1, T / WKV7_CHUNK), D, D], dtype: .float32)
    try check(rwkv_wkv7_train_fwd(r.raw, w.raw, k.raw, v.raw, a.raw, b.raw, r.dtype.code, hIn?.f32, out.f32, hOut.f32,
                                  sa.f32, ck.f32, Int64(B), Int64(T), Int64(H), streamArg))
    return (out, hOut, WKV7TrainSaved(sa: sa, hCkpt: ck, hIn: hIn))
}

/// WKV7Train.swift:472-475.
public func wkv7Train(_ r: DeviceArray, _ w: DeviceArray, _ k: DeviceArray, _ v: DeviceArray,
                      _ a: DeviceArray, _ b: DeviceArray) throws -> DeviceArray {
    try wkv7TrainWithState(r, w, k, v, a, b, nil).0
}

/// The VJP of wkv7TrainWithState (WKV7Train.swift:426-467): cotangents of
/// (out, h_out) (nil h_out cotangent = zeros) → gradients of r, w, k, v, a,
/// b in each primal's dtype (:440,462) and of h_in in fp32.
public func wkv7TrainBackward(_ r: DeviceArray, _ w: DeviceArray, _ k: DeviceArray, _ v: DeviceArray,
                              _ a: DeviceArray, _ b: DeviceArray, saved: WKV7TrainSaved,
                              dOut: DeviceArray, dHOut: DeviceArray?) throws -> ([DeviceArray], DeviceArray) {
    let (B, T, H) = try btph(r)
    let D = WKV7_HEAD_SIZE
    let grads = try (0 ..< 6).map { _ in try DeviceArray(shape: [B, T, H, D], dtype: r.dtype) }
    let dh = try DeviceArray(shape: [B, H, D, D], dtype: .float32)
    try check(rwkv_wkv7_train_bwd(r.raw, w.raw, k.raw, v.raw, a.raw, b.raw, r.dtype.code, saved.hIn?.f32,
                                  saved.hCkpt.f32, saved.sa.f32, dOut.f32, dHOut?.f32, grads[0].raw, grads[1].raw,
                                  grads[2].raw, grads[3].raw, grads[4].raw, grads[5].raw, r.dtype.code, dh.f32,
                                  Int64(B), Int64(T), Int64(H), wkv7BackwardV2 ? 2 : 1, streamArg))
    return (grads, dh)
}

/// WKV7DecodeKernels.swift:73-89 — one token; r..b [H, 64], h [H, 64, 64].
public func wkv7StepForward(_ r: DeviceArray, _ w: DeviceArray, _ k: DeviceArray, _ v: DeviceArray,
                            _ a: DeviceArray, _ b: DeviceArray, _ h: DeviceArray) throws -> (DeviceArray, DeviceArray) {
    guard r.shape.count == 2, r.shape[1] == WKV7_HEAD_SIZE,
          h.shape == [r.shape[0], WKV7_HEAD_SIZE, WKV7_HEAD_SIZE] else {
        throw RWKVHipError.status(Int32(RWKV_E_SHAPE.rawValue), "step: r \(r.shape), state \(h.shape)")
    }
    let H = r.shape[0]
    let out = try DeviceArray(shape: [H, WKV7_HEAD_SIZE], dtype: .float32)
    let hOut = try DeviceArray(shape: h.shape, dtype: .float32)
    try check(rwkv_wkv7_step(r.raw, w.raw, k.raw, v.raw, a.raw, b.raw, r.dtype.code, h.f32, out.f32, hOut.f32, 1,
                             Int64(H), streamArg))
    return (out, hOut)
}

/// WKV7DecodeKernels.swift:92.
public func wkvTailApplies(headSize S: Int) -> Bool { rwkv_wkv_tail_applies(Int64(S)) != 0 }

/// WKV7DecodeKernels.swift:106-178 — group norm, bonus and gate over N rows.
public func wkvTail(_ wkv: DeviceArray, r: DeviceArray, k: DeviceArray, v: DeviceArray, rK: DeviceArray,
                    lnWeight: DeviceArray, lnBias: DeviceArray, gate: DeviceArray, nHead H: Int, headSize S: Int,
                    rows N: Int = 1, eps: Float = 64e-5) throws -> DeviceArray {
    let out = try DeviceArray(shape: [N, H * S], dtype: .float32)
    try check(rwkv_wkv_tail(wkv.f32, r.f32, k.f32, v.f32, rK.f32, lnWeight.f32, lnBias.f32, gate.f32, out.f32,
                            Int64(N), Int64(H), Int64(S), eps, streamArg))
    return out
}

/// The tmix decode step's wkv7StepForward + wkvTail pair (X070Generation.swift:280-295)
/// as one launch for B rows, state updated in place.
public func wkv7StepTailInPlace(_ r: DeviceArray, _ w: DeviceArray, _ k: DeviceArray, _ v: DeviceArray,
                                _ a: DeviceArray, _ b: DeviceArray, state: DeviceArray, rK: DeviceArray,
                                lnWeight: DeviceArray, lnBias: DeviceArray, gate: DeviceArray,
                                eps: Float = 64e-5) throws -> DeviceArray {
    let (B, H) = (state.shape[0], state.shape[1])
    let out = try DeviceArray(shape: [B, H * WKV7_HEAD_SIZE], dtype: .float32)
    try check(rwkv_wkv7_step_tail(r.f32, w.f32, k.f32, v.f32, a.f32, b.f32, state.f32, state.f32, rK.f32, lnWeight.f32,
                                  lnBias.f32, gate.f32, nil, out.f32, Int64(B), Int64(H), eps, streamArg))
    return out
}
