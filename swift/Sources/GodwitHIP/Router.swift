import CGodwitHIP
import Foundation

/// Selects which experts a token needs (Runtime/Router.swift:11-104): router
/// logits on the device, top-k and the softmax over the k on the host.
public struct Router {
    /// One token's routing decision (:13-23).
    public struct Decision: Sendable, Equatable {
        /// Chosen expert ids, highest logit first.
        public let experts: [Int]
        /// Softmax over the selected logits only — not over all experts.
        public let weights: [Float]

        public init(experts: [Int], weights: [Float]) {
            self.experts = experts
            self.weights = weights
        }
    }

    public let context: HIPContext
    public let expertCount: Int
    public let hiddenSize: Int
    public let topK: Int

    public init(context: HIPContext, expertCount: Int, hiddenSize: Int, topK: Int) {
        self.context = context
        self.expertCount = expertCount
        self.hiddenSize = hiddenSize
        self.topK = topK
    }

    /// Router logits for one token (:38-66): bf16 weight [experts, hidden] and
    /// bias [experts] resident on the device, fp16 hidden state.  Blocks.
    public func logits(
        for hidden: [Float16], weight: GWBuffer, bias: GWBuffer
    ) throws -> [Float] {
        precondition(hidden.count == hiddenSize, "expected \(hiddenSize) inputs")
        let x = try context.buffer(hidden)
        let output = try context.emptyBuffer(of: Float.self, count: expertCount)
        try check(gw_router_logits(context.handle, weight.ptr, GW_BF16, bias.ptr, GW_BF16, x.ptr,
                                   GW_F16, output.ptr.assumingMemoryBound(to: Float.self),
                                   Int64(expertCount), Int64(hiddenSize), 1))
        return try output.download(Float.self, count: expertCount)
    }

    /// Turns logits into a routing decision (:78-98): top-k by partial
    /// selection sort first, then the softmax over only those k logits.  Runs
    /// on the host (gw_router_select), as the reference's does.
    public func select(logits: [Float]) -> Decision {
        precondition(logits.count == expertCount, "expected \(expertCount) logits")
        var ids = [Int32](repeating: 0, count: topK)
        var weights = [Float](repeating: 0, count: topK)
        let status = logits.withUnsafeBufferPointer { l in
            ids.withUnsafeMutableBufferPointer { i in
                weights.withUnsafeMutableBufferPointer { w in
                    gw_router_select(l.baseAddress, Int64(expertCount), Int64(topK),
                                     i.baseAddress, w.baseAddress)
                }
            }
        }
        precondition(status == 0, String(cString: gw_last_error()))
        return Decision(experts: ids.map { Int($0) }, weights: weights)
    }

    /// logits(for:weight:bias:) then select(logits:) (:100-104).
    public func route(
        hidden: [Float16], weight: GWBuffer, bias: GWBuffer
    ) throws -> Decision {
        select(logits: try logits(for: hidden, weight: weight, bias: bias))
    }
}
