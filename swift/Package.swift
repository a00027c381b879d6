// swift-tools-version:5.9
// The Swift side of Godwit's MoE path over libgodwit_hip (the C ABI in
// include/godwit_hip.h).  CGodwitHIP is the system-library target for the C
// header and the shared library; GodwitHIP keeps the reference engine's
// ExpertRunner / Router / Decision surface on top of it.
//
//   swift build -Xlinker -L<directory of libgodwit_hip.so>
import PackageDescription

let package = Package(
    name: "GodwitHIP",
    products: [
        .library(name: "GodwitHIP", targets: ["GodwitHIP"]),
    ],
    targets: [
        .systemLibrary(name: "CGodwitHIP", path: "Sources/CGodwitHIP"),
        .target(name: "GodwitHIP", dependencies: ["CGodwitHIP"], path: "Sources/GodwitHIP"),
    ]
)
