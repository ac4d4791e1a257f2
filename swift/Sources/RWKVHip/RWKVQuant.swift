// RWKVQuant over the MI355X C ABI: the .rwkvq container and manifest
// (RwkvqFile.swift / RwkvqSidecar.swift), the fused dequant kernels
// (RwkvqDequant.swift) and the decode GEMVs with their applicability tables
// and nil-return fallbacks (RwkvqSb6GEMV.swift, RwkvqSymGEMV.swift), plus the
// matrix-core long pass of baseMatmul (X070Backbone.swift:337-356).

import CRwkvHip

public enum RwkvqKind: Int32 {
    case dense = 0, sb6 = 1, sym = 2, asym = 3, rtn = 4   // rwkvq_kind
}

/// RwkvqError (RwkvqSidecar.swift:25-56), from the reader's findings.
public enum RwkvqError: Error {
    case missingFile(String)
    case malformedManifest(String)
    case missingBuffer(tensor: String, buffer: String)
    case shapeMismatch(tensor: String, expected: [Int], got: [Int])
}

/// RwkvqTensorInfo (RwkvqSidecar.swift:75-99).
public struct RwkvqTensorInfo {
    public let kind: RwkvqKind
    public let shape: [Int]
    public let bits: Int
    public let xbits: Int
    public let groupSize: Int
    public let superBlock: Int
    public let packed: Bool
    public let outlierCount: Int
    public let transposed: Bool
    public var outFeatures: Int { shape[0] }
    public var inFeatures: Int { shape[1] }
}

/// An opened .rwkvq file with its validated manifest; the K3 / sym-interleave
/// layouts are read straight from the mapping (rwkvq_read_sb6 / _sym).
public final class RwkvqFileHandle {
    let file: OpaquePointer
    let manifest: OpaquePointer
    public private(set) var tensors: [String: RwkvqTensorInfo] = [:]
    private var index: [String: Int64] = [:]
    public let nLayer: Int, nEmbd: Int, headSize: Int, vocabSize: Int
    public let naming: String

    /// RwkvqSidecar.maxFormatVersion.
    public static let maxFormatVersion: Int32 = 2

    public init(path: String) throws {
        var f: OpaquePointer? = nil
        let st = rwkvq_open(path, &f)
        guard st == RWKV_OK, let fh = f else {
            let msg = String(cString: rwkv_last_error())
            throw st == RWKV_E_IO ? RwkvqError.missingFile(msg) : RwkvqError.malformedManifest(msg)
        }
        var m: OpaquePointer? = nil
        var finding = rwkvq_finding()
        guard rwkvq_manifest_read(fh, Self.maxFormatVersion, &m, &finding) == RWKV_OK, let mh = m else {
            rwkvq_close(fh)
            let msg = String(cString: rwkv_last_error())
            let tensor = withUnsafeBytes(of: finding.tensor) { String(cString: $0.bindMemory(to: CChar.self).baseAddress!) }
            let buffer = withUnsafeBytes(of: finding.buffer) { String(cString: $0.bindMemory(to: CChar.self).baseAddress!) }
            switch finding.kind {
            case Int32(RWKVQ_FINDING_MISSING_BUFFER.rawValue): throw RwkvqError.missingBuffer(tensor: tensor, buffer: buffer)
            case Int32(RWKVQ_FINDING_SHAPE.rawValue):
                let e = withUnsafeBytes(of: finding.expected) { Array($0.bindMemory(to: Int64.self)) }
                let g = withUnsafeBytes(of: finding.got) { Array($0.bindMemory(to: Int64.self)) }
                throw RwkvqError.shapeMismatch(tensor: tensor, expected: e.prefix(Int(finding.n_expected)).map { Int($0) },
                                               got: g.prefix(Int(finding.n_got)).map { Int($0) })
            default: throw RwkvqError.malformedManifest(msg)
            }
        }
        file = fh
        manifest = mh
        var model = rwkvq_model()
        _ = rwkvq_manifest_model(mh, &model)
        nLayer = Int(model.n_layer); nEmbd = Int(model.n_embd)
        headSize = Int(model.head_size); vocabSize = Int(model.vocab_size)
        naming = String(cString: model.naming)
        var d = rwkvq_tensor()
        for i in 0 ..< rwkvq_manifest_count(mh) {
            _ = rwkvq_manifest_tensor(mh, i, &d)
            let key = String(cString: d.key)
            let shape = withUnsafeBytes(of: d.shape) { Array($0.bindMemory(to: Int64.self)) }
            index[key] = i
            tensors[key] = RwkvqTensorInfo(kind: RwkvqKind(rawValue: d.kind) ?? .dense,
                                           shape: shape.prefix(Int(d.ndim)).map { Int($0) }, bits: Int(d.bits),
                                           xbits: Int(d.xbits), groupSize: Int(d.group_size),
                                           superBlock: Int(d.super_block), packed: d.packed != 0,
                                           outlierCount: Int(d.outliers), transposed: d.transposed != 0)
        }
    }

    deinit {
        rwkvq_manifest_free(manifest)
        rwkvq_close(file)
    }

    /// The loader layout of an sb6 matrix on the device: (qblk, qsqm, ddm).
    public func sb6Buffers(_ key: String) throws -> (DeviceArray, DeviceArray, DeviceArray) {
        guard let info = tensors[key], info.kind == .sb6, let i = index[key] else {
            throw RwkvqError.missingBuffer(tensor: key, buffer: "qblk")
        }
        let (O, I) = (info.outFeatures, info.inFeatures)
        var qblk = [UInt8](repeating: 0, count: O * I / 32 * (16 + 4 * info.xbits))
        var qsqm = [UInt8](repeating: 0, count: O * I / 16)
        var ddm = [UInt16](repeating: 0, count: O * I / 128)
        try check(rwkvq_read_sb6(file, manifest, i, &qblk, &qsqm, &ddm))
        return (try DeviceArray.upload(qblk, shape: [O, qblk.count / O], dtype: .uint8),
                try DeviceArray.upload(qsqm, shape: [O, I / 16], dtype: .uint8),
                try DeviceArray.upload(ddm, shape: [O, I / 128], dtype: .float16))
    }

    /// The loader layout of a sym matrix on the device: (qblk, qs, d).
    public func symBuffers(_ key: String) throws -> (DeviceArray, DeviceArray, DeviceArray) {
        guard let info = tensors[key], info.kind == .sym, let i = index[key] else {
            throw RwkvqError.missingBuffer(tensor: key, buffer: "qblk")
        }
        let (O, I) = (info.outFeatures, info.inFeatures)
        var qblk = [UInt8](repeating: 0, count: info.bits == 8 ? O * I : O * I / 32 * 24)
        var qs = [UInt8](repeating: 0, count: O * I / 16)
        var d = [UInt16](repeating: 0, count: O * I / 256)
        try check(rwkvq_read_sym(file, manifest, i, &qblk, &qs, &d))
        return (try DeviceArray.upload(qblk, shape: [O, qblk.count / O], dtype: .uint8),
                try DeviceArray.upload(qs, shape: [O, I / 16], dtype: .uint8),
                try DeviceArray.upload(d, shape: [O, I / 256], dtype: .float16))
    }
}

// ───────────────────────────── dequant ─────────────────────────────

/// RwkvqDequant.swift:160-183 — packed sb6 → dense [OUT, IN] (combine in fp32).
public func rwkvqDequantDense(qblk: DeviceArray, qsqm: DeviceArray, ddm: DeviceArray, outFeatures OUT: Int,
                              inFeatures IN: Int, superBlock: Int, xbits: Int,
                              dtype: DeviceDType = .float32) throws -> DeviceArray {
    guard superBlock == 8 else {
        throw RWKVHipError.status(Int32(RWKV_E_UNSUPPORTED.rawValue), "sb6 dequant is built for super-block 8")
    }
    let out = try DeviceArray(shape: [OUT, IN], dtype: dtype)
    try check(rwkv_sb6_dequant(qblk.u8, qsqm.u8, ddm.u16, out.raw, dtype.code, Int64(OUT), Int64(IN), Int32(xbits),
                               streamArg))
    return out
}

/// RwkvqDequant.swift:409-466 — sym → dense, any IN of whole 16-column blocks.
public func rwkvqDequantSym(qblk: DeviceArray, qs: DeviceArray, d: DeviceArray, outFeatures OUT: Int,
                            inFeatures IN: Int, bits: Int, dtype: DeviceDType = .float32) throws -> DeviceArray {
    let out = try DeviceArray(shape: [OUT, IN], dtype: dtype)
    try check(rwkv_sym_dequant(qblk.u8, qs.u8, d.u16, out.raw, dtype.code, Int64(OUT), Int64(IN), Int32(bits),
                               streamArg))
    return out
}

// ───────────────────────────── decode GEMV ─────────────────────────────

/// RwkvqSb6GEMV.swift:159-164 — the reference's table, rows == 1 included.
public func rwkvqSb6GEMVApplies(outFeatures OUT: Int, inFeatures IN: Int, xbits: Int, superBlock: Int,
                                rows: Int) -> Bool {
    rwkv_sb6_gemv_applies(Int64(OUT), Int64(IN), Int32(xbits), Int32(superBlock), Int64(rows)) != 0
}

/// RwkvqSb6GEMV.swift:170-190 — y [N, OUT] = x [N, IN]·Wᵀ from the K3 bytes (fp32).
/// N rows share one weight pass (the reference launches N = 1).
public func rwkvqSb6GEMV(_ x: DeviceArray, qblk: DeviceArray, qsqm: DeviceArray, ddm: DeviceArray,
                         outFeatures OUT: Int, inFeatures IN: Int, xbits: Int) throws -> DeviceArray {
    guard x.shape.count == 2, x.shape[1] == IN, x.dtype == .float32 else {
        throw RWKVHipError.status(Int32(RWKV_E_SHAPE.rawValue), "sb6-GEMV: input \(x.shape), expected [N, \(IN)] fp32")
    }
    let y = try DeviceArray(shape: [x.shape[0], OUT], dtype: .float32)
    try check(rwkv_sb6_gemv(x.f32, Int64(x.shape[0]), qblk.u8, qsqm.u8, ddm.u16, y.f32, Int64(OUT), Int64(IN),
                            Int32(xbits), streamArg))
    return y
}

/// RwkvqSymGEMV.swift:213-218.
public func rwkvqSymGEMVApplies(outFeatures OUT: Int, inFeatures IN: Int, bits: Int, rows: Int) -> Bool {
    rwkv_sym_gemv_applies(Int64(OUT), Int64(IN), Int32(bits), Int64(rows)) != 0
}

/// RwkvqSymGEMV.swift:223-247 (outPer = OUT) and symGEMVFused (:343-358,
/// outPer < OUT: row o of input n reads x[n·K + o / outPer]).
public func rwkvqSymGEMV(_ x: DeviceArray, qblk: DeviceArray, qs: DeviceArray, d: DeviceArray,
                         outFeatures OUT: Int, inFeatures IN: Int, bits: Int, outPer: Int? = nil) throws -> DeviceArray {
    let per = outPer ?? OUT
    let K = OUT / per
    let N = x.shape[0] / K
    let y = try DeviceArray(shape: [N, OUT], dtype: .float32)
    try check(rwkv_sym_gemv(x.f32, Int64(N), qblk.u8, qs.u8, d.u16, y.f32, Int64(OUT), Int64(IN), Int32(bits),
                            Int64(per), streamArg))
    return y
}

/// The sidecar wrappers with the reference's nil fallbacks
/// (RwkvqSb6GEMV.swift:197-208, RwkvqSymGEMV.swift:254-263): nil when the
/// kernel does not take the shape, so the caller dequantises instead.
public final class RwkvqDeviceSidecar {
    public let file: RwkvqFileHandle
    public private(set) var arrays: [String: (DeviceArray, DeviceArray, DeviceArray)] = [:]

    public init(path: String, only: ((String) -> Bool)? = nil) throws {
        file = try RwkvqFileHandle(path: path)
        for (key, info) in file.tensors where only?(key) ?? true {
            switch info.kind {
            case .sb6: arrays[key] = try file.sb6Buffers(key)
            case .sym: arrays[key] = try file.symBuffers(key)
            default: break
            }
        }
    }

    public func sb6GEMV(_ key: String, _ x: DeviceArray) throws -> DeviceArray? {
        guard let info = file.tensors[key], info.kind == .sb6, x.shape.count == 2, x.shape[1] == info.inFeatures,
              rwkvqSb6GEMVApplies(outFeatures: info.outFeatures, inFeatures: info.inFeatures, xbits: info.xbits,
                                  superBlock: info.superBlock, rows: x.shape[0]),
              let (qblk, qsqm, ddm) = arrays[key] else { return nil }
        return try rwkvqSb6GEMV(x, qblk: qblk, qsqm: qsqm, ddm: ddm, outFeatures: info.outFeatures,
                                inFeatures: info.inFeatures, xbits: info.xbits)
    }

    public func symGEMV(_ key: String, _ x: DeviceArray) throws -> DeviceArray? {
        guard let info = file.tensors[key], info.kind == .sym, x.shape.count == 2, x.shape[1] == info.inFeatures,
              rwkvqSymGEMVApplies(outFeatures: info.outFeatures, inFeatures: info.inFeatures, bits: info.bits,
                                  rows: x.shape[0]),
              let (qblk, qs, d) = arrays[key] else { return nil }
        return try rwkvqSymGEMV(x, qblk: qblk, qs: qs, d: d, outFeatures: info.outFeatures,
                                inFeatures: info.inFeatures, bits: info.bits)
    }

    /// The split-K workspace a long pass of M rows takes (nil: one K range).
    private func gemmWorkspace(_ M: Int, _ info: RwkvqTensorInfo) throws -> (DeviceArray?, Int64) {
        let n = rwkv_quant_gemm_workspace(Int64(M), Int64(info.outFeatures), Int64(info.inFeatures))
        return n > 0 ? (try DeviceArray(shape: [Int(n)], dtype: .uint8), n) : (nil, 0)
    }

    /// The long pass of baseMatmul with an fp16 base (X070Backbone.swift:337-356):
    /// y = fp16(fp16(x)·fp16(W)ᵀ) on the matrix cores from the packed bytes;
    /// nil where the kernel does not take the matrix (the caller dequantises).
    public func sb6LongPass(_ key: String, _ x: DeviceArray) throws -> DeviceArray? {
        guard let info = file.tensors[key], info.kind == .sb6, x.shape.count == 2,
              x.shape[1] == info.inFeatures, x.dtype == .float32 || x.dtype == .float16,
              rwkv_sb6_gemm_applies(Int64(info.outFeatures), Int64(info.inFeatures), Int32(info.xbits),
                                    Int64(info.outFeatures)) != 0,
              let (qblk, qsqm, ddm) = arrays[key] else { return nil }
        let M = x.shape[0]
        let y = try DeviceArray(shape: [M, info.outFeatures], dtype: .float32)
        let (ws, wsBytes) = try gemmWorkspace(M, info)
        try check(rwkv_sb6_gemm(x.raw, x.dtype.code, Int64(M), Int64(info.inFeatures), Int64(M * info.inFeatures),
                                qblk.u8, qsqm.u8, ddm.u16, y.raw, Int64(info.outFeatures), Int64(info.outFeatures),
                                Int64(info.inFeatures), Int32(info.xbits), Int64(info.outFeatures), 0,
                                ws?.raw, wsBytes, streamArg))
        return y
    }

    /// sb6LongPass for a sym matrix (8-bit codes or the 6-bit interleave):
    /// fp16(W) is the fp16 branch of rwkvqDequantSym (RwkvqDequant.swift:350-388).
    public func symLongPass(_ key: String, _ x: DeviceArray) throws -> DeviceArray? {
        guard let info = file.tensors[key], info.kind == .sym, x.shape.count == 2,
              x.shape[1] == info.inFeatures, x.dtype == .float32 || x.dtype == .float16,
              rwkv_sym_gemm_applies(Int64(info.outFeatures), Int64(info.inFeatures), Int32(info.bits),
                                    Int64(info.outFeatures)) != 0,
              let (qblk, qs, d) = arrays[key] else { return nil }
        let M = x.shape[0]
        let y = try DeviceArray(shape: [M, info.outFeatures], dtype: .float32)
        let (ws, wsBytes) = try gemmWorkspace(M, info)
        try check(rwkv_sym_gemm(x.raw, x.dtype.code, Int64(M), Int64(info.inFeatures), Int64(M * info.inFeatures),
                                qblk.u8, qs.u8, d.u16, y.raw, Int64(info.outFeatures), Int64(info.outFeatures),
                                Int64(info.inFeatures), Int32(info.bits), Int64(info.outFeatures), 0,
                                ws?.raw, wsBytes, streamArg))
        return y
    }
}
