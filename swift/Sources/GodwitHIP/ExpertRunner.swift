import CGodwitHIP
import Foundation

/// Owns one gw_expert_runner and the per-runner staging the single-token calls
/// use; destroyed with the last ExpertRunner value that holds it.
final class RunnerHandle {
    let context: HIPContext
    let runner: OpaquePointer   // gw_expert_runner *
    let input: GWBuffer         // one token's fp16 hidden state
    let output: GWBuffer        // one token's fp32 result

    init(context: HIPContext, hiddenSize: Int, intermediateSize: Int,
         activation: FeedForwardActivation, limit: Float, alpha: Float) throws {
        var h: OpaquePointer?
        try check(gw_expert_runner_create(context.handle, Int64(hiddenSize),
                                          Int64(intermediateSize), activation.cValue, limit,
                                          alpha, &h))
        runner = h!
        self.context = context
        do {
            input = try context.emptyBuffer(of: Float16.self, count: hiddenSize)
            output = try context.emptyBuffer(of: Float.self, count: hiddenSize)
        } catch {
            _ = gw_expert_runner_destroy(h)
            throw error
        }
    }

    deinit { _ = gw_expert_runner_destroy(runner) }
}

/// Runs one expert's feed-forward branch — gate_up projection, interleaved
/// gated activation, down projection — and the routed combinations of several
/// (Runtime/ExpertRunner.swift:10-363), on libgodwit_hip's HIP kernels.
public struct ExpertRunner {
    public let context: HIPContext
    public let reader: ModelReader
    public let hiddenSize: Int
    public let intermediateSize: Int
    public let swigluLimit: Float
    public let swigluAlpha: Float
    /// The reference switches between two Metal GEMV geometries; the HIP
    /// kernels have one (every decode kernel runs a fixed, balanced grid), so
    /// this is kept for source compatibility and has no effect.
    public var usePersistentKernel = true
    /// Kept for source compatibility with the Metal runner; not used.
    public static let persistentThreadgroups = 64

    let handle: RunnerHandle

    /// ExpertRunner.init (:37-47).  The limit and alpha default to the
    /// model's activationLimit / activationAlpha.  Throws where the reference
    /// cannot fail: creating the runner allocates its device scratch.
    public init(context: HIPContext, reader: ModelReader,
                swigluLimit: Float? = nil, swigluAlpha: Float? = nil) throws {
        self.context = context
        self.reader = reader
        let spec = reader.manifest.spec
        self.hiddenSize = spec.hiddenSize
        self.intermediateSize = spec.intermediateSize
        self.swigluLimit = swigluLimit ?? spec.activationLimit
        self.swigluAlpha = swigluAlpha ?? spec.activationAlpha
        self.handle = try RunnerHandle(context: context, hiddenSize: spec.hiddenSize,
                                       intermediateSize: spec.intermediateSize,
                                       activation: spec.activation,
                                       limit: self.swigluLimit, alpha: self.swigluAlpha)
    }

    /// One expert as a single device buffer plus the offsets of its six
    /// sub-tensors (:54-64).
    public struct Weights {
        public let buffer: GWBuffer
        public let offsets: [ExpertLayout.Section: Int]

        public init(buffer: GWBuffer, offsets: [ExpertLayout.Section: Int]) {
            self.buffer = buffer
            self.offsets = offsets
        }

        func offset(_ section: ExpertLayout.Section) -> Int { offsets[section] ?? 0 }

        /// The C ABI's gw_expert_weights for this expert.
        var cValue: gw_expert_weights {
            var c = gw_expert_weights()
            c.buffer = UnsafePointer(buffer.ptr.assumingMemoryBound(to: UInt8.self))
            c.offsets = (Int64(offset(.gateUpBlocks)), Int64(offset(.gateUpScales)),
                         Int64(offset(.downBlocks)), Int64(offset(.downScales)),
                         Int64(offset(.gateUpBias)), Int64(offset(.downBias)))
            return c
        }
    }

    /// Section offsets within an expert stride, from the manifest (:67-75).
    public var sectionOffsets: [ExpertLayout.Section: Int] {
        var result: [ExpertLayout.Section: Int] = [:]
        for section in ExpertLayout.Section.allCases {
            if let span = reader.manifest.expertSections[section.rawValue] {
                result[section] = span.offset
            }
        }
        return result
    }

    /// Reads one expert into fresh device memory, bypassing any cache (:77-86).
    public func loadWeights(layer: Int, expert: Int) throws -> Weights {
        let buffer = try reader.loadExpertStride(layer: layer, expert: expert, context: context)
        return Weights(buffer: buffer, offsets: sectionOffsets)
    }

    /// One expert's work for one token (:88-98).
    public struct Assignment {
        public let weights: Weights
        public let token: Int
        public let routingWeight: Float

        public init(weights: Weights, token: Int, routingWeight: Float) {
            self.weights = weights
            self.token = token
            self.routingWeight = routingWeight
        }
    }

    /// Applies many (expert, token) pairs, accumulating into per-token outputs
    /// (:108-182): outputs[token] += routingWeight * expert(inputs[token]).
    /// inputs: fp16 [tokens, hidden]; outputs: fp32 [tokens, hidden], which the
    /// caller zero-fills first.  Each distinct expert is read once per group
    /// of up to 8 tokens.  Blocks until the outputs are complete.
    public func applyAssignments(
        inputs: GWBuffer, assignments: [Assignment], outputs: GWBuffer
    ) throws {
        guard !assignments.isEmpty else { return }
        let table = assignments.map { a -> gw_assignment in
            precondition(a.token >= 0, "negative token index")
            return gw_assignment(weights: a.weights.cValue, token: Int32(a.token),
                                 routing_weight: a.routingWeight)
        }
        try table.withUnsafeBufferPointer { list in
            try check(gw_expert_apply_assignments(
                handle.runner, inputs.ptr, GW_F16, list.baseAddress, Int32(list.count),
                outputs.ptr.assumingMemoryBound(to: Float.self)))
        }
    }

    /// Applies every selected expert to one token and combines them in list
    /// order on the device (:191-269).  No experts: zeros, as the reference.
    public func applyBatch(
        _ input: [Float16], experts: [(weights: Weights, weight: Float)]
    ) throws -> [Float] {
        precondition(input.count == hiddenSize, "expected \(hiddenSize) inputs")
        guard !experts.isEmpty else { return [Float](repeating: 0, count: hiddenSize) }
        try handle.input.upload(input)
        let weights = experts.map { $0.weights.cValue }
        let routing = experts.map { $0.weight }
        try weights.withUnsafeBufferPointer { w in
            try routing.withUnsafeBufferPointer { r in
                try check(gw_expert_apply_batch(
                    handle.runner, handle.input.ptr, GW_F16, w.baseAddress, r.baseAddress,
                    Int32(experts.count), handle.output.ptr.assumingMemoryBound(to: Float.self)))
            }
        }
        return try handle.output.download(Float.self, count: hiddenSize)
    }

    /// Applies one expert to a single token's hidden state, before any routing
    /// weight (:275-331).
    public func apply(_ input: [Float16], weights: Weights) throws -> [Float] {
        precondition(input.count == hiddenSize, "expected \(hiddenSize) inputs")
        try handle.input.upload(input)
        var w = weights.cValue
        try check(gw_expert_apply(handle.runner, handle.input.ptr, GW_F16, &w,
                                  handle.output.ptr.assumingMemoryBound(to: Float.self)))
        return try handle.output.download(Float.self, count: hiddenSize)
    }
}

extension ExpertRunner {
    /// TransformerLayer.forward's MoE block (Runtime/TransformerLayer.swift:
    /// 158-230) on the device in one call: route (from `logits`, or from the
    /// router weights when `logits` is nil), run each selected expert, combine
    /// in router order into `out` (fp32 [tokens, hidden], overwritten).  One
    /// token runs as one kernel; larger batches as grouped GEMMs.  Enqueues
    /// only; `context.synchronize()` waits.
    public func moeLayer(
        layer: GWBuffer, topK: Int, x: GWBuffer, tokens: Int, out: GWBuffer,
        logits: GWBuffer? = nil, routerWeight: GWBuffer? = nil, routerBias: GWBuffer? = nil,
        outBF16: GWBuffer? = nil, routingIDs: GWBuffer? = nil, routingWeights: GWBuffer? = nil
    ) throws {
        var args = gw_moe_layer_args()
        args.experts_base = UnsafePointer(layer.ptr.assumingMemoryBound(to: UInt8.self))
        args.expert_stride = Int64(reader.manifest.expertStride)
        args.expert_count = Int64(reader.manifest.expertCount)
        args.top_k = Int64(topK)
        args.logits = logits.map { UnsafePointer($0.ptr.assumingMemoryBound(to: Float.self)) }
        args.router_weight = routerWeight.map { UnsafeRawPointer($0.ptr) }
        args.router_weight_dtype = GW_BF16
        args.router_bias = routerBias.map { UnsafeRawPointer($0.ptr) }
        args.router_bias_dtype = GW_BF16
        args.x = UnsafeRawPointer(x.ptr)
        args.x_dtype = GW_F16
        args.tokens = Int32(tokens)
        args.out = out.ptr.assumingMemoryBound(to: Float.self)
        args.out_bf16 = outBF16.map { $0.ptr.assumingMemoryBound(to: UInt16.self) }
        args.routing_ids = routingIDs.map { $0.ptr.assumingMemoryBound(to: Int32.self) }
        args.routing_weights = routingWeights.map { $0.ptr.assumingMemoryBound(to: Float.self) }
        try check(gw_moe_layer_forward(handle.runner, &args))
    }

    /// Sizes the batched path's scratch up front, as a caller about to capture
    /// a graph must (nothing may be allocated during capture).
    public func reservePrefill(maxTokens: Int, topK: Int) throws {
        try check(gw_expert_runner_reserve_prefill(handle.runner, Int32(maxTokens), Int32(topK),
                                                   Int32(reader.manifest.expertCount)))
    }

    /// Waves of the one-token layer kernel whose bounded wait for the other
    /// workgroups gave up since the runner was created (0 while every result
    /// is valid).  When one gives up, the next `context.synchronize()` throws
    /// GodwitHIPError with status GW_ERR_EXCHANGE once, and the runner runs
    /// later one-token layers as two kernels.  Blocks on the stream.
    public func syncErrors() throws -> Int {
        var n: UInt32 = 0
        try check(gw_expert_runner_sync_errors(handle.runner, &n))
        return Int(n)
    }

    /// Polls of the one-token layer's exchange before a wait gives up (0: the
    /// default, 2^18).
    public func setWaitLimit(_ polls: UInt32) throws {
        try check(gw_expert_runner_set_wait_limit(handle.runner, polls))
    }
}
