// swift-tools-version:5.9
// SwiftPM package of the Swift side of the MI355X path: the reference's
// RWKVKernel / RWKVQuant entry points (same names, argument meaning and
// fallback rules) over the C ABI of libswiftrwkv_hip.so (include/rwkv_hip.h).
// Build on a ROCm host:  swift build -Xlinker -L<repo>/swiftrwkv_amd -Xcc -I/opt/rocm/include
//                                    -Xlinker -L/opt/rocm/lib
import PackageDescription

let package = Package(
    name: "RWKVHip",
    products: [.library(name: "RWKVHip", targets: ["RWKVHip"])],
    targets: [
        .target(
            name: "CRwkvHip",
            path: "Sources/CRwkvHip",
            cSettings: [.define("__HIP_PLATFORM_AMD__"), .unsafeFlags(["-I/opt/rocm/include"])],
            linkerSettings: [.linkedLibrary("swiftrwkv_hip"), .linkedLibrary("amdhip64")]),
        .target(name: "RWKVHip", dependencies: ["CRwkvHip"], path: "Sources/RWKVHip"),
    ])
