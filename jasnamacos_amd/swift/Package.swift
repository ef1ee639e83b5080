// swift-tools-version: 5.9
// libdcn for Swift hosts: the CDCN system-library target (the C ABI of include/dcn/dcn.h),
// the HIPDeformConv runner (MetalDeformConv's surface, MetalRunner.swift:92-185) and a
// self-test executable. To bind the reference package instead, add the CDCN target and
// the linker settings below to its manifest (Package.swift:1-17), make JasnaMetalPoC
// depend on "CDCN", and drop Sources/HIPDeformConv/HIPDeformConv.swift beside
// MetalRunner.swift (the reference's own DeformConvShape / DeformConvError then replace
// ReferenceInterface.swift).
import Foundation
import PackageDescription

let here = URL(fileURLWithPath: #filePath).deletingLastPathComponent()
let libDir = here.deletingLastPathComponent().appendingPathComponent("lib").path  // jasnamacos_amd/lib
let linkLibdcn: [LinkerSetting] = [.unsafeFlags(["-L", libDir, "-Xlinker", "-rpath", "-Xlinker", libDir])]

let package = Package(
    name: "DCNHIP",
    products: [
        .library(name: "HIPDeformConv", targets: ["HIPDeformConv"]),
        .executable(name: "dcn-self-test", targets: ["dcn-self-test"]),
    ],
    targets: [
        .systemLibrary(name: "CDCN", path: "Sources/CDCN"),
        .target(name: "HIPDeformConv", dependencies: ["CDCN"], linkerSettings: linkLibdcn),
        .executableTarget(name: "dcn-self-test", dependencies: ["HIPDeformConv", "CDCN"], linkerSettings: linkLibdcn),
    ]
)
