// Device buffers for the Swift side of the MI355X path.
//
// MLX has no ROCm backend, so on an MI355X host the arrays the reference
// keeps as MLXArray live here as DeviceArray: one hipMalloc'ed buffer, its
// shape and element type.  Ownership follows the reference's value
// semantics: every entry point returns new arrays and never writes its
// inputs (the in-place decode entries say so in their names).

import CRwkvHip

public enum RWKVHipError: Error, CustomStringConvertible {
    /// A non-OK rwkv_status with the library's message (the reference traps
    /// on these preconditions; here they are thrown).
    case status(Int32, String)
    case hip(String)

    public var description: String {
        switch self {
        case .status(let s, let m): return "rwkv_status \(s): \(m)"
        case .hip(let m): return "HIP: \(m)"
        }
    }
}

@inline(__always)
func check(_ s: rwkv_status) throws {
    guard s == RWKV_OK else {
        throw RWKVHipError.status(Int32(s.rawValue), String(cString: rwkv_last_error()))
    }
}

/// Element types the entry points take (rwkv_dtype), plus the byte buffers
/// of the quantised layouts.
public enum DeviceDType: Equatable {
    case float32, bfloat16, float16, uint8, int32

    public var size: Int {
        switch self {
        case .float32, .int32: return 4
        case .bfloat16, .float16: return 2
        case .uint8: return 1
        }
    }

    var code: rwkv_dtype {
        switch self {
        case .bfloat16: return RWKV_BF16
        case .float16: return RWKV_F16
        default: return RWKV_F32
        }
    }
}

/// A device array: `count` elements of `dtype`, row-major in `shape`.
public final class DeviceArray {
    public let shape: [Int]
    public let dtype: DeviceDType
    public let raw: UnsafeMutableRawPointer
    private let owned: Bool

    public var count: Int { shape.reduce(1, *) }
    public var nbytes: Int { count * dtype.size }

    public init(shape: [Int], dtype: DeviceDType) throws {
        self.shape = shape
        self.dtype = dtype
        var p: UnsafeMutableRawPointer? = nil
        let n = max(1, shape.reduce(1, *) * dtype.size)
        guard hipMalloc(&p, n) == hipSuccess, let q = p else { throw RWKVHipError.hip("hipMalloc(\(n)) failed") }
        raw = q
        owned = true
    }

    /// A view of rows [start, start + rows) of a row-major array (the row
    /// slices of a fused group); it does not own the memory.
    public init(viewOf base: DeviceArray, rowStart start: Int, rows: Int) {
        let rowElems = base.shape.dropFirst().reduce(1, *)
        shape = [rows] + Array(base.shape.dropFirst())
        dtype = base.dtype
        raw = base.raw + start * rowElems * base.dtype.size
        owned = false
    }

    deinit { if owned { hipFree(raw) } }

    public static func zeros(_ shape: [Int], dtype: DeviceDType = .float32) throws -> DeviceArray {
        let a = try DeviceArray(shape: shape, dtype: dtype)
        guard hipMemset(a.raw, 0, a.nbytes) == hipSuccess else { throw RWKVHipError.hip("hipMemset failed") }
        return a
    }

    /// Host bytes → a new device array (synchronous).
    public static func upload<T>(_ host: [T], shape: [Int], dtype: DeviceDType) throws -> DeviceArray {
        let a = try DeviceArray(shape: shape, dtype: dtype)
        precondition(host.count * MemoryLayout<T>.stride == a.nbytes, "upload: \(host.count) elements for \(shape)")
        try host.withUnsafeBytes { b in
            guard hipMemcpy(a.raw, b.baseAddress, a.nbytes, hipMemcpyHostToDevice) == hipSuccess else {
                throw RWKVHipError.hip("hipMemcpy H2D failed")
            }
        }
        return a
    }

    /// Device → host (synchronous).
    public func download<T>(as: T.Type) throws -> [T] {
        var out = [T](unsafeUninitializedCapacity: nbytes / MemoryLayout<T>.stride) { _, n in
            n = nbytes / MemoryLayout<T>.stride
        }
        try out.withUnsafeMutableBytes { b in
            guard hipMemcpy(b.baseAddress, raw, nbytes, hipMemcpyDeviceToHost) == hipSuccess else {
                throw RWKVHipError.hip("hipMemcpy D2H failed")
            }
        }
        return out
    }

    var f32: UnsafeMutablePointer<Float> { raw.assumingMemoryBound(to: Float.self) }
    var u8: UnsafeMutablePointer<UInt8> { raw.assumingMemoryBound(to: UInt8.self) }
    var u16: UnsafeMutablePointer<UInt16> { raw.assumingMemoryBound(to: UInt16.self) }
    var i32: UnsafeMutablePointer<Int32> { raw.assumingMemoryBound(to: Int32.self) }
}

/// The stream every call is enqueued on (nil = the default stream), as the
/// reference's calls go to MLX's default stream.
nonisolated(unsafe) public var rwkvHipStream: hipStream_t? = nil

var streamArg: UnsafeMutableRawPointer? { rwkvHipStream.map { UnsafeMutableRawPointer($0) } }
