// swift-tools-version: 5.9
// MXQ: the quantized-linear operators of the reference's MLX-Swift surface
// (quantized, dequantized, quantizedMatmul / quantizedMM, QuantizedLinear, MfLinear),
// running on libmxq.so (HIP, gfx950) through its C ABI, include/mxq.h.
//
// Build against an in-tree libmxq.so:
//   swift build -Xlinker -L<repo>/wuxianhuabu_amd -Xlinker -rpath -Xlinker <repo>/wuxianhuabu_amd
// A host package depends on it as the reference's package depends on mlx-swift
// (`Packages/z-image-swift/Package.swift:21-33`):
//   .package(path: "<repo>/wuxianhuabu_amd/swift"), then .product(name: "MXQ", package: "MXQ")
import PackageDescription

let package = Package(
    name: "MXQ",
    products: [
        .library(name: "MXQ", targets: ["MXQ"]),
    ],
    targets: [
        // the C ABI: include/mxq.h through a module map; links libmxq
        .systemLibrary(name: "CMXQ", path: "Sources/CMXQ"),
        .target(name: "MXQ", dependencies: ["CMXQ"], path: "Sources/MXQ"),
    ]
)
