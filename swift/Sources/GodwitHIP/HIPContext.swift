import CGodwitHIP
import Foundation

/// A failed libgodwit_hip call: its status and the library's message.
///
/// Takes the place of the reference's `MetalError` cases and of its
/// `precondition` traps on shapes, which the C ABI reports as statuses.
public struct GodwitHIPError: Error, CustomStringConvertible {
    public let status: Int32
    public let message: String

    public var description: String { "godwit_hip status \(status): \(message)" }
}

/// Throws unless `status` is GW_OK, with gw_last_error()'s message.
@inline(__always)
func check(_ status: Int32) throws {
    guard status == 0 else {
        throw GodwitHIPError(status: status, message: String(cString: gw_last_error()))
    }
}

/// One GPU and the stream every call on it is ordered on (MetalContext,
/// Infrastructure/Metal/MetalContext.swift:36-179: device + command queue).
public final class HIPContext {
    let handle: OpaquePointer   // gw_context *

    public init(device: Int = 0) throws {
        var h: OpaquePointer?
        try check(gw_context_create(Int32(device), &h))
        handle = h!
    }

    deinit { _ = gw_context_destroy(handle) }

    /// Waits for everything enqueued on the context (MetalContext.run's wait).
    /// Throws GW_ERR_EXCHANGE (status 7) once when a one-token layer's bounded
    /// wait gave up since the last call (that layer's outputs are invalid; see
    /// ExpertRunner.syncErrors).
    public func synchronize() throws { try check(gw_context_synchronize(handle)) }

    /// MetalContext.buffer(_:): a device copy of `values`.
    public func buffer<T>(_ values: [T]) throws -> GWBuffer {
        let b = try GWBuffer(context: self, length: max(1, values.count * MemoryLayout<T>.stride))
        try b.upload(values)
        return b
    }

    /// MetalContext.emptyBuffer(of:count:): uninitialised device memory.
    public func emptyBuffer<T>(of type: T.Type, count: Int) throws -> GWBuffer {
        try GWBuffer(context: self, length: max(1, count * MemoryLayout<T>.stride))
    }
}

/// Device memory from gw_malloc, freed with its owner (stands in for MTLBuffer).
public final class GWBuffer {
    public let context: HIPContext
    public let ptr: UnsafeMutableRawPointer
    public let length: Int

    public init(context: HIPContext, length: Int) throws {
        var p: UnsafeMutableRawPointer?
        try check(gw_malloc(context.handle, length, &p))
        guard let q = p else {
            throw GodwitHIPError(status: Int32(GW_ERR_ARG.rawValue), message: "empty allocation")
        }
        self.context = context
        self.ptr = q
        self.length = length
    }

    deinit { _ = gw_free(context.handle, ptr) }

    /// Host -> device, blocking, at byte `offset`.
    public func upload<T>(_ values: [T], offset: Int = 0) throws {
        try values.withUnsafeBytes { raw in
            precondition(offset + raw.count <= length, "upload past the end of the buffer")
            guard let base = raw.baseAddress, raw.count > 0 else { return }
            try check(gw_memcpy_htod(context.handle, ptr + offset, base, raw.count))
        }
    }

    /// Device -> host, blocking (MTLBuffer.contents() after the wait).
    public func download<T>(_ type: T.Type, count: Int, offset: Int = 0) throws -> [T] {
        let bytes = count * MemoryLayout<T>.stride
        precondition(offset + bytes <= length, "download past the end of the buffer")
        let staging = UnsafeMutableRawPointer.allocate(byteCount: max(1, bytes),
                                                       alignment: MemoryLayout<T>.alignment)
        defer { staging.deallocate() }
        if bytes > 0 {
            try check(gw_memcpy_dtoh(context.handle, staging, ptr + offset, bytes))
        }
        let typed = staging.bindMemory(to: T.self, capacity: count)
        return Array(UnsafeBufferPointer(start: typed, count: count))
    }
}
