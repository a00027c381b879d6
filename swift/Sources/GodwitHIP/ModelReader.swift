import CGodwitHIP
import Foundation

/// The six sub-tensors of one expert stride (ExpertLayout.Section,
/// Install/InstallLayout.swift:18-24); raw values are the manifest's names.
public enum ExpertLayout {
    public enum Section: String, CaseIterable {
        case gateUpBlocks = "gate_up_blocks"
        case gateUpScales = "gate_up_scales"
        case downBlocks = "down_blocks"
        case downScales = "down_scales"
        case gateUpBias = "gate_up_bias"
        case downBias = "down_bias"

        /// Index in the C ABI's section order (GW_SECTION_*).
        var index: Int {
            switch self {
            case .gateUpBlocks: return 0
            case .gateUpScales: return 1
            case .downBlocks: return 2
            case .downScales: return 3
            case .gateUpBias: return 4
            case .downBias: return 5
            }
        }
    }
}

/// FeedForwardActivation (Model/ArchitectureSpec.swift:14-38), as the C ABI
/// names the two expert activations.
public enum FeedForwardActivation {
    case gptOssClampedGLU
    case silu

    var cValue: gw_activation {
        switch self {
        case .gptOssClampedGLU: return GW_ACT_GPTOSS_CLAMPED_GLU
        case .silu: return GW_ACT_SILU
        }
    }
}

/// The manifest fields the MoE path reads (GodwitManifest,
/// Install/GodwitManifest.swift:8-105), decoded by gw_model_open.
public struct Manifest {
    public struct Span { public let offset: Int; public let length: Int }

    public struct Spec {
        public let hiddenSize: Int
        public let intermediateSize: Int
        public let rmsNormEpsilon: Float
        public let activation: FeedForwardActivation
        public let activationLimit: Float
        public let activationAlpha: Float
        public let expertBias: Bool
        public let routerBias: Bool
        public let expertsPerToken: Int
    }

    public let formatVersion: Int
    public let layerCount: Int
    public let expertCount: Int
    public let expertStride: Int
    public let expertSections: [String: Span]
    public let spec: Spec

    init(_ info: gw_model_info) {
        formatVersion = Int(info.format_version)
        layerCount = Int(info.layer_count)
        expertCount = Int(info.expert_count)
        expertStride = Int(info.expert_stride)
        var sections: [String: Span] = [:]
        withUnsafeBytes(of: info.section_offset) { offsets in
            withUnsafeBytes(of: info.section_length) { lengths in
                let o = offsets.bindMemory(to: Int64.self)
                let l = lengths.bindMemory(to: Int64.self)
                for section in ExpertLayout.Section.allCases {
                    sections[section.rawValue] = Span(offset: Int(o[section.index]),
                                                      length: Int(l[section.index]))
                }
            }
        }
        expertSections = sections
        spec = Spec(hiddenSize: Int(info.hidden_size),
                    intermediateSize: Int(info.intermediate_size),
                    rmsNormEpsilon: info.rms_norm_epsilon,
                    activation: info.activation == GW_ACT_SILU ? .silu : .gptOssClampedGLU,
                    activationLimit: info.activation_limit,
                    activationAlpha: info.activation_alpha,
                    expertBias: info.expert_bias != 0,
                    routerBias: info.router_bias != 0,
                    expertsPerToken: Int(info.experts_per_token))
    }
}

/// A .gwt installation (ModelReader, Runtime/ModelReader.swift:11-111): the
/// manifest, and expert strides or whole layer files read into device memory
/// (pread into pinned staging, copied by the context's stream).
public final class ModelReader {
    public let directory: URL
    public let manifest: Manifest
    let handle: OpaquePointer   // gw_model *

    /// ModelReader.init (:17-37): manifest required, format version 2.
    public init(directory: URL) throws {
        var h: OpaquePointer?
        try check(gw_model_open(directory.path, &h))
        var info = gw_model_info()
        let status = gw_model_info_get(h, &info)
        if status != 0 {
            _ = gw_model_close(h)
            try check(status)
        }
        self.handle = h!
        self.directory = directory
        self.manifest = Manifest(info)
    }

    deinit { _ = gw_model_close(handle) }

    /// GodwitManifest.validate (:79-104): every layer file has the size the
    /// manifest implies.
    public func validate() throws { try check(gw_model_validate(handle)) }

    /// ModelReader.loadExpertStride(layer:expert:device:) (:72-90): one expert's
    /// whole stride in fresh device memory.
    public func loadExpertStride(layer: Int, expert: Int, context: HIPContext) throws -> GWBuffer {
        let buffer = try GWBuffer(context: context, length: manifest.expertStride)
        try check(gw_model_load_expert(context.handle, handle, Int32(layer), Int32(expert),
                                       buffer.ptr))
        return buffer
    }

    /// A whole layer file (expertCount strides), the experts_base of the layer
    /// entry points.
    public func loadLayer(_ layer: Int, context: HIPContext) throws -> GWBuffer {
        let bytes = manifest.expertStride * manifest.expertCount
        let buffer = try GWBuffer(context: context, length: bytes)
        try check(gw_model_load_layer(context.handle, handle, Int32(layer), buffer.ptr, bytes))
        return buffer
    }
}
