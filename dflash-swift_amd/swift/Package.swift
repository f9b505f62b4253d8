// swift-tools-version:5.9
//
// DFlashKitHIP: the Swift surface of DFlashKit's small-M quantised matmul
// (Sources/DFlashKit/SmallMQuantizedMatmul.swift in the reference) over the MI355X C ABI of
// include/dflash_qmm.h.  Build libdflash_qmm.so first (make -C dflash-swift_amd) and point
// the linker at it, e.g.
//
//     swift build -Xlinker -L$(pwd)/../dflash_qmm -Xlinker -rpath -Xlinker $(pwd)/../dflash_qmm
//
import PackageDescription

let package = Package(
    name: "DFlashKitHIP",
    products: [
        .library(name: "DFlashKitHIP", targets: ["DFlashKitHIP"])
    ],
    targets: [
        // The C ABI: include/dflash_qmm.h, linked against libdflash_qmm.so.
        .systemLibrary(name: "CDFlashQMM", path: "Sources/CDFlashQMM"),
        .target(name: "DFlashKitHIP", dependencies: ["CDFlashQMM"], path: "Sources/DFlashKitHIP"),
    ]
)
