//
//  SmallMQuantizedMatmulHIP.swift
//  DFlashKitHIP
//
//  DFlashKit's small-M quantised matmul surface -- SmallMQuantizedMatmul, SmallMQuantizedLinear
//  and enableSmallMQuantizedMatmul(in:), Sources/DFlashKit/SmallMQuantizedMatmul.swift:27-317 in
//  the reference -- on a ROCm host, over the MI355X (gfx950) kernels of libdflash_qmm.so and its
//  C ABI (include/dflash_qmm.h).
//
//  The reference subclasses MLX's QuantizedLinear and walks MLX's module tree.  MLX has no HIP
//  backend, so this module carries the two pieces of that framework the path touches, reduced
//  to what the swap needs: a device array (any host framework's array with a device address
//  conforms to `DeviceArray`) and a module tree of named children (`Module`).  The public names,
//  the eligibility window, the fall-through rule and the swap are the reference's.
//

import CDFlashQMM

// MARK: - Errors

/// A dfq_* call returned a non-zero status.
public struct DFQError: Error, CustomStringConvertible {
    public let status: dfq_status
    public let call: String
    public let message: String

    public init(status: dfq_status, call: String, message: String) {
        self.status = status
        self.call = call
        self.message = message
    }

    /// The error of the failed call `call`, with the library's message for it (read on the
    /// thread that made the call).
    public init(status: dfq_status, call: String) {
        self.init(status: status, call: call, message: String(cString: dfq_last_error()))
    }

    public var description: String { "\(call): status \(status.rawValue): \(message)" }
}

/// Throws the call's error unless it returned DFQ_OK.
@inline(__always)
public func check(_ status: dfq_status, _ call: String) throws {
    if status != DFQ_OK { throw DFQError(status: status, call: call) }
}

/// Failures inside a forward are programming or device errors with no recovery path; the
/// reference stops the process for its one such case too (a missing kernel variant,
/// SmallMQuantizedMatmul.swift:214-216).
@inline(__always)
func mustSucceed(_ status: dfq_status, _ call: String) {
    if status != DFQ_OK {
        preconditionFailure("\(call): status \(status.rawValue): \(String(cString: dfq_last_error()))")
    }
}

// MARK: - Device arrays

/// Element types of the arrays the path reads and writes.
public enum DeviceDType: Equatable {
    case bfloat16, float16, float32, uint32

    /// Bytes per element.
    public var size: Int {
        switch self {
        case .bfloat16, .float16: return 2
        case .float32, .uint32: return 4
        }
    }

    var dfq: dfq_dtype {
        switch self {
        case .bfloat16: return DFQ_BF16
        case .float16: return DFQ_F16
        case .float32: return DFQ_F32
        case .uint32: preconditionFailure("uint32 is the packed-weight type, not a float dtype")
        }
    }

    init(_ d: dfq_dtype) {
        switch d {
        case DFQ_BF16: self = .bfloat16
        case DFQ_F16: self = .float16
        default: self = .float32
        }
    }
}

/// A row-major array in device memory of the context's GPU: the role MLXArray plays in the
/// reference.  Any host framework's array type with a device address can conform.
public protocol DeviceArray: AnyObject {
    var deviceAddress: UnsafeMutableRawPointer { get }
    var shape: [Int] { get }
    var dtype: DeviceDType { get }
}

extension DeviceArray {
    /// Number of elements.
    public var count: Int { shape.reduce(1, *) }

    /// The same memory seen with another shape of the same element count.
    public func reshaped(_ shape: [Int]) -> DeviceArray {
        precondition(shape.reduce(1, *) == count, "reshape must keep the element count")
        return DeviceView(base: self, shape: shape)
    }
}

/// Device memory allocated by this module (layer outputs), taken from and returned to its
/// context's pool: no device allocation or free happens on a warm forward path.
public final class DeviceBuffer: DeviceArray {
    public let deviceAddress: UnsafeMutableRawPointer
    public let shape: [Int]
    public let dtype: DeviceDType
    let context: HIPContext
    private let bytes: Int

    public init(context: HIPContext, shape: [Int], dtype: DeviceDType) throws {
        let bytes = DevicePool.sizeClass(max(1, shape.reduce(1, *) * dtype.size))
        self.deviceAddress = try context.pool.take(bytes)
        self.bytes = bytes
        self.shape = shape
        self.dtype = dtype
        self.context = context
    }

    deinit {
        context.pool.give(deviceAddress, bytes)
    }
}

/// A stream-ordered cache of device blocks for one context.  Every call of a context runs on
/// its one stream, so a block handed back when its last user's array goes away can serve the
/// next array at once: any kernel that writes it through the new array is queued after every
/// kernel that used it through the old one.  Blocks come in power-of-two sizes from 256
/// bytes up and go back to the device only when the context ends.  Used from one thread at
/// a time, as the generator serialises its work on one queue
/// (DFlashSpeculativeGenerator.swift:93-99).  For eager forwards: a captured HIP graph
/// keeps the addresses it recorded, so code that captures the layers' calls manages those
/// buffers itself (the C ABI's dfq_graph_* over caller-owned memory).
final class DevicePool {
    private let handle: OpaquePointer
    private var free: [Int: [UnsafeMutableRawPointer]] = [:]
    private var all: [UnsafeMutableRawPointer] = []

    init(handle: OpaquePointer) { self.handle = handle }

    static func sizeClass(_ bytes: Int) -> Int {
        var c = 256
        while c < bytes { c <<= 1 }
        return c
    }

    func take(_ bytes: Int) throws -> UnsafeMutableRawPointer {
        if let p = free[bytes]?.popLast() { return p }
        var p: UnsafeMutableRawPointer?
        try check(dfq_malloc(handle, bytes, &p), "dfq_malloc")
        all.append(p!)
        return p!
    }

    func give(_ p: UnsafeMutableRawPointer, _ bytes: Int) {
        free[bytes, default: []].append(p)
    }

    /// Frees every block; the stream must be idle.
    func drain() {
        for p in all { _ = dfq_free(handle, p) }
        all = []
        free = [:]
    }
}

/// A reshaped view that keeps its base alive.
final class DeviceView: DeviceArray {
    let base: DeviceArray
    let shape: [Int]
    var deviceAddress: UnsafeMutableRawPointer { base.deviceAddress }
    var dtype: DeviceDType { base.dtype }

    init(base: DeviceArray, shape: [Int]) {
        self.base = base
        self.shape = shape
    }
}

// MARK: - The GPU context

/// One GPU: the loaded gfx950 code object (dfq_init), a stream, and the workspaces of the
/// matmuls issued on it.  MLX's default device and stream play this role in the reference.
public final class HIPContext {
    public let handle: OpaquePointer
    /// The hipStream_t every call of this context is issued on.
    public let stream: UnsafeMutableRawPointer?
    /// Workspaces as raw (address, bytes): the last is current, older ones stay until the
    /// context goes, since work queued on the stream may still use them.  Raw, not
    /// DeviceBuffer, so that they hold no reference back to the context.
    private var workspaces: [(UnsafeMutableRawPointer, Int)] = []
    /// Device blocks of the arrays this context's layers return.
    let pool: DevicePool
    /// The greedy accept's device buffers for a verify width: its workspace (zero at rest:
    /// cleared once when made, every call leaves it zero), the tokens with the accepted count
    /// behind them, and the proposals.  Raw for the same reason as the workspaces.
    var acceptBuffers: [Int: (ws: UnsafeMutableRawPointer, wsBytes: Int,
                              out: UnsafeMutableRawPointer, props: UnsafeMutableRawPointer)] = [:]

    /// The context layers use unless they are given one.
    public static let shared: HIPContext = {
        do {
            return try HIPContext(device: 0)
        } catch {
            preconditionFailure("no usable MI355X for the small-M quantised matmul: \(error)")
        }
    }()

    public init(device: Int32) throws {
        var h: OpaquePointer?
        try check(dfq_init(device, &h), "dfq_init")
        var s: UnsafeMutableRawPointer?
        let st = dfq_stream_create(h, &s)
        if st != DFQ_OK {
            let message = String(cString: dfq_last_error())
            _ = dfq_destroy(h)
            throw DFQError(status: st, call: "dfq_stream_create", message: message)
        }
        self.handle = h!
        self.stream = s
        self.pool = DevicePool(handle: h!)
    }

    deinit {
        _ = dfq_stream_sync(handle, stream)
        for (p, _) in workspaces { _ = dfq_free(handle, p) }
        for b in acceptBuffers.values {
            _ = dfq_free(handle, b.ws)
            _ = dfq_free(handle, b.out)
            _ = dfq_free(handle, b.props)
        }
        pool.drain()
        _ = dfq_stream_destroy(handle, stream)
        _ = dfq_destroy(handle)
    }

    /// A workspace of at least `bytes` as (address, bytes), zero at rest (cleared on the
    /// stream when created; every matmul leaves it zero again), or nil when none is needed.
    func workspace(_ bytes: Int) -> (UnsafeMutableRawPointer, Int)? {
        if bytes == 0 { return nil }
        if let ws = workspaces.last, ws.1 >= bytes { return ws }
        let size = max(bytes, 1 << 20)
        var p: UnsafeMutableRawPointer?
        mustSucceed(dfq_malloc(handle, size, &p), "dfq_malloc")
        mustSucceed(dfq_workspace_clear(handle, p, size, stream), "dfq_workspace_clear")
        workspaces.append((p!, size))
        return (p!, size)
    }

    /// Waits until everything issued on the context's stream has run.
    public func synchronize() throws {
        try check(dfq_stream_sync(handle, stream), "dfq_stream_sync")
    }
}

// MARK: - The module tree

/// A module tree reduced to what the swap needs: named children, leaves by dotted path, and
/// replacement of modules at paths (MLXNN's leafModules().flattened() and
/// update(modules:), used by the reference at SmallMQuantizedMatmul.swift:305-315).
open class Module {
    public private(set) var children: [(String, Module)] = []

    public init() {}

    /// Adds or replaces the child called `name`.
    public func setChild(_ name: String, _ module: Module) {
        if let i = children.firstIndex(where: { $0.0 == name }) {
            children[i].1 = module
        } else {
            children.append((name, module))
        }
    }

    /// Every module without children, with its dotted path.
    public func leafModules() -> [(String, Module)] {
        var out: [(String, Module)] = []
        for (name, child) in children {
            if child.children.isEmpty {
                out.append((name, child))
            } else {
                out += child.leafModules().map { ("\(name).\($0.0)", $0.1) }
            }
        }
        return out
    }

    /// Replaces the modules at the given dotted paths.
    public func update(modules: [(String, Module)]) {
        for (path, module) in modules {
            var parts = path.split(separator: ".").map(String.init)
            let last = parts.removeLast()
            var node: Module = self
            for p in parts {
                guard let next = node.children.first(where: { $0.0 == p })?.1 else {
                    preconditionFailure("no module at \(path)")
                }
                node = next
            }
            node.setChild(last, module)
        }
    }
}

// MARK: - The stock layer

/// MLX's QuantizedLinear over device arrays: weight uint32 [out][in * bits / 32] (element 0 in
/// the low bits), scales and biases [out][in / groupSize], an optional linear bias [out].
/// Every forward runs the stock path (dfq_qmm_fallback: a GEMV for few rows), the stand-in
/// for MLX's quantizedMatmul that SmallMQuantizedLinear falls through to
/// (SmallMQuantizedMatmul.swift:265).
open class QuantizedLinear: Module {
    public enum Mode: Equatable { case affine, mxfp4 }

    public let weight: DeviceArray
    public let bias: DeviceArray?
    public let scales: DeviceArray
    public let biases: DeviceArray?
    public let groupSize: Int
    public let bits: Int
    public let mode: Mode
    public let context: HIPContext

    /// (output features, input features).
    public var shape: (Int, Int) { (weight.shape[0], weight.shape[1] * 32 / bits) }

    public init(weight: DeviceArray, bias: DeviceArray?, scales: DeviceArray,
                biases: DeviceArray?, groupSize: Int, bits: Int, mode: Mode = .affine,
                context: HIPContext = .shared) {
        self.weight = weight
        self.bias = bias
        self.scales = scales
        self.biases = biases
        self.groupSize = groupSize
        self.bits = bits
        self.mode = mode
        self.context = context
        super.init()
    }

    /// MLX's type promotion of the input with the scales: equal dtypes keep it, else fp32.
    func outputDType(_ x: DeviceDType) -> DeviceDType { x == scales.dtype ? x : .float32 }

    open func callAsFunction(_ x: DeviceArray) -> DeviceArray {
        guard mode == .affine, let biases else {
            preconditionFailure("the stock path here handles the affine mode with biases")
        }
        let (outputFeatures, inputFeatures) = shape
        let rows = x.count / inputFeatures
        let ydt = outputDType(x.dtype)
        guard let y = try? DeviceBuffer(context: context,
                                        shape: Array(x.shape.dropLast()) + [outputFeatures],
                                        dtype: ydt) else {
            preconditionFailure("output allocation failed")
        }
        mustSucceed(dfq_qmm_fallback(context.handle, x.deviceAddress,
                                     weight.deviceAddress.assumingMemoryBound(to: UInt32.self),
                                     scales.deviceAddress, biases.deviceAddress,
                                     bias?.deviceAddress, y.deviceAddress, Int32(rows),
                                     Int32(outputFeatures), Int32(inputFeatures), Int32(bits),
                                     Int32(groupSize), x.dtype.dfq, scales.dtype.dfq, ydt.dfq,
                                     context.stream),
                    "dfq_qmm_fallback")
        return y
    }
}

// MARK: - The kernel's window and launch

/// The reference's enum: the eligibility window (SmallMQuantizedMatmul.swift:29-49, the same
/// constants the C ABI exports), isEligible (:193-201), tiles(for:) (:205-207) and apply
/// (:210-224), which here launches dfq_qmm on the context's stream.
enum SmallMQuantizedMatmul {
    static let minimumRows = Int(DFQ_MINIMUM_ROWS)
    static let maximumRows = Int(DFQ_MAXIMUM_ROWS)
    /// Also read by the generator's width snapping (DFlashSpeculativeGenerator.swift:136-142,
    /// 325-326).
    static let rowsPerTile = Int(DFQ_ROWS_PER_TILE)
    static let minimumOutputFeatures = Int(DFQ_MINIMUM_OUTPUT_FEATURES)
    static let inputFeatureMultiple = Int(DFQ_INPUT_FEATURE_MULTIPLE)
    static let requiredGroupSize = Int(DFQ_REQUIRED_GROUP_SIZE)

    /// The gate's shape-and-format half (affine with biases, 4 or 8 bits, group 64, at least
    /// 4096 outputs, inputs a multiple of 512), which no row count changes: the swap asks it
    /// once per layer, the forward never.
    static func isEligible(_ layer: QuantizedLinear) -> Bool {
        let (outputFeatures, inputFeatures) = layer.shape
        return dfq_is_eligible(Int32(outputFeatures), Int32(inputFeatures), Int32(layer.bits),
                               Int32(layer.groupSize), layer.mode == .affine ? 1 : 0,
                               layer.biases == nil ? 0 : 1) == 1
    }

    /// Row tiles of `rowsPerTile` a launch of `rows` rows computes: 1 for 1...8, 2 for 9...16.
    static func tiles(for rows: Int) -> Int { Int(dfq_tiles_for(Int32(rows))) }

    /// y[rows, N] = x[rows, K] . dequant(w)^T (+ bias), bf16, on the fast kernel.  No padding
    /// rows are needed: the kernel stores only the rows it is given.
    static func apply(x: DeviceArray, weight: DeviceArray, scales: DeviceArray,
                      biases: DeviceArray, bias: DeviceArray?, rows: Int, outputFeatures: Int,
                      inputFeatures: Int, bits: Int, context: HIPContext) -> DeviceArray {
        let h = context.handle
        var need = 0
        mustSucceed(dfq_qmm_workspace_bytes(h, Int32(rows), Int32(outputFeatures),
                                            Int32(inputFeatures), Int32(bits),
                                            Int32(requiredGroupSize), &need),
                    "dfq_qmm_workspace_bytes")
        let ws = context.workspace(need)
        guard let y = try? DeviceBuffer(context: context, shape: [rows, outputFeatures],
                                        dtype: .bfloat16) else {
            preconditionFailure("output allocation failed")
        }
        mustSucceed(dfq_qmm(h, x.deviceAddress,
                            weight.deviceAddress.assumingMemoryBound(to: UInt32.self),
                            scales.deviceAddress, biases.deviceAddress, bias?.deviceAddress,
                            y.deviceAddress, Int32(rows), Int32(outputFeatures),
                            Int32(inputFeatures), Int32(bits), Int32(requiredGroupSize),
                            DFQ_BF16, DFQ_BF16, DFQ_BF16, ws?.0, ws?.1 ?? 0, context.stream),
                    "dfq_qmm")
        return y
    }

    /// ``apply`` over a weight in the packed layout (dfq_qmm_packed).
    static func applyPacked(x: DeviceArray, packed: DeviceArray, bias: DeviceArray?, rows: Int,
                            outputFeatures: Int, inputFeatures: Int, bits: Int,
                            context: HIPContext) -> DeviceArray {
        let h = context.handle
        var need = 0
        mustSucceed(dfq_qmm_workspace_bytes(h, Int32(rows), Int32(outputFeatures),
                                            Int32(inputFeatures), Int32(bits),
                                            Int32(requiredGroupSize), &need),
                    "dfq_qmm_workspace_bytes")
        let ws = context.workspace(need)
        guard let y = try? DeviceBuffer(context: context, shape: [rows, outputFeatures],
                                        dtype: .bfloat16) else {
            preconditionFailure("output allocation failed")
        }
        mustSucceed(dfq_qmm_packed(h, x.deviceAddress, packed.deviceAddress,
                                   bias?.deviceAddress, y.deviceAddress, Int32(rows),
                                   Int32(outputFeatures), Int32(inputFeatures), Int32(bits),
                                   Int32(requiredGroupSize), DFQ_BF16, ws?.0, ws?.1 ?? 0,
                                   context.stream),
                    "dfq_qmm_packed")
        return y
    }
}

// MARK: - The drop-in layer

/// The drop-in layer (SmallMQuantizedMatmul.swift:234-293): the same arrays as the layer it
/// wraps; a forward whose row count lies in the window goes to the MI355X kernel, any other
/// forward to the stock path, unchanged.
public final class SmallMQuantizedLinear: QuantizedLinear {

    /// The gate's static half for this layer, computed when the layer is built (:236-240),
    /// so that a caller who wraps an ineligible layer by hand still gets the stock result.
    private let kernelEligible: Bool
    /// Row counts of the window the fast kernel has a work split for at this shape (none for
    /// weights of 2 GiB or more); other rows take the stock path like an ineligible call.
    private let kernelRows: Set<Int>
    /// The weight, scales and biases again in the packed layout, once ``packWeights()`` has
    /// built it: the window's calls then read it instead of the three arrays.
    public private(set) var packed: DeviceBuffer?

    /// The drop-in over `other`'s own weight, scale, bias and linear-bias arrays: nothing is
    /// copied, so swapping adds no weight memory (:243-252).
    public init(_ other: QuantizedLinear) {
        let eligible = SmallMQuantizedMatmul.isEligible(other)
        var fits = Set<Int>()
        if eligible {
            let (n, k) = other.shape
            for rows in SmallMQuantizedMatmul.minimumRows...SmallMQuantizedMatmul.maximumRows
            where dfq_qmm_supported(other.context.handle, Int32(rows), Int32(n), Int32(k),
                                    Int32(other.bits), Int32(other.groupSize), DFQ_BF16,
                                    DFQ_BF16, DFQ_BF16) == 1 {
                fits.insert(rows)
            }
        }
        self.kernelEligible = eligible
        self.kernelRows = fits
        super.init(weight: other.weight, bias: other.bias, scales: other.scales,
                   biases: other.biases, groupSize: other.groupSize, bits: other.bits,
                   mode: other.mode, context: other.context)
    }

    /// Opt-in: a second copy of this layer's weight, scales and biases in the packed layout
    /// (dfq_pack_weights), which the fast kernel reads as whole cache lines (bit-identical
    /// results, about 0.3-0.7 us less per call at the 17408 x 5120 shape on MI355X).  The
    /// stock path keeps using the arrays, so the layer then holds its weight twice.  Throws
    /// for a layer the window never serves or whose input width is not a whole number of
    /// 8-group chunks.  Not in the reference, which reads MLX's arrays in place.
    public func packWeights() throws {
        guard packed == nil else { return }
        guard kernelEligible, scales.dtype == .bfloat16, let biases else {
            throw DFQError(status: DFQ_ERR_UNSUPPORTED, call: "packWeights",
                           message: "a packed copy serves the window's bf16 calls only")
        }
        let (n, k) = shape
        var bytes = 0
        try check(dfq_packed_bytes(Int32(n), Int32(k), Int32(bits), Int32(groupSize), &bytes),
                  "dfq_packed_bytes")
        // whole 16-byte units: the buffer's words are the packed layout's bytes
        let buffer = try DeviceBuffer(context: context, shape: [bytes / 4], dtype: .uint32)
        try check(dfq_pack_weights(context.handle,
                                   weight.deviceAddress.assumingMemoryBound(to: UInt32.self),
                                   scales.deviceAddress, biases.deviceAddress, Int32(n),
                                   Int32(k), Int32(bits), Int32(groupSize),
                                   buffer.deviceAddress, context.stream),
                  "dfq_pack_weights")
        packed = buffer
    }

    public override func callAsFunction(_ x: DeviceArray) -> DeviceArray {
        let shape = x.shape
        let rows = shape.dropLast().reduce(1, *)
        // The kernel writes bf16 from bf16 inputs.  An fp16 input, whose stock result MLX
        // promotes to fp32, must keep getting exactly that, so it falls through (:258-266).
        guard kernelEligible,
            rows >= SmallMQuantizedMatmul.minimumRows,
            rows <= SmallMQuantizedMatmul.maximumRows,
            kernelRows.contains(rows),
            x.dtype == .bfloat16, scales.dtype == .bfloat16,
            let biases
        else {
            return super.callAsFunction(x)
        }
        let inputFeatures = shape[shape.count - 1]
        let outputFeatures = weight.shape[0]
        if let packed {
            return SmallMQuantizedMatmul.applyPacked(
                x: x, packed: packed, bias: bias, rows: rows, outputFeatures: outputFeatures,
                inputFeatures: inputFeatures, bits: bits, context: context
            ).reshaped(Array(shape.dropLast()) + [outputFeatures])
        }
        // the linear bias is fused into the kernel's store (the reference's `y + bias`, :288-290)
        let y = SmallMQuantizedMatmul.apply(
            x: x, weight: weight, scales: scales, biases: biases, bias: bias, rows: rows,
            outputFeatures: outputFeatures, inputFeatures: inputFeatures, bits: bits,
            context: context)
        return y.reshaped(Array(shape.dropLast()) + [outputFeatures])
    }
}

/// Replaces each leaf of `model` that is a ``QuantizedLinear`` passing the static gate, and
/// is not already a drop-in, by a ``SmallMQuantizedLinear`` over the same arrays
/// (SmallMQuantizedMatmul.swift:303-317).  The caller opts in: the kernel sums in another
/// order than the stock path, so swapped layers' outputs move by about one bf16 ulp.
///
/// - Returns: the number of leaves replaced (0 on a second call).
@discardableResult
public func enableSmallMQuantizedMatmul(in model: Module) -> Int {
    let updates = model
        .leafModules()
        .compactMap { (path, module) -> (String, Module)? in
            guard !(module is SmallMQuantizedLinear),
                let quantized = module as? QuantizedLinear,
                SmallMQuantizedMatmul.isEligible(quantized)
            else { return nil }
            return (path, SmallMQuantizedLinear(quantized))
        }
    model.update(modules: updates)
    return updates.count
}

// MARK: - The fused MLP

extension HIPContext {
    /// At load: `out` gets the gate and up arrays interleaved in blocks of 8 rows (rows
    /// 16t...16t+7 are gate rows 8t...8t+7, rows 16t+8...16t+15 the matching up rows), the
    /// layout of gateUpSiLU's weights.  Call it for the weight (rowBytes = K * bits / 8), the
    /// scales and the biases (rowBytes = K / groupSize * 2) and a linear bias (2).
    public func interleaveGateUp(gate: UnsafeRawPointer, up: UnsafeRawPointer,
                                 out: UnsafeMutableRawPointer, hidden: Int,
                                 rowBytes: Int) throws {
        try check(dfq_interleave_gate_up(handle, gate, up, out, Int32(hidden), rowBytes,
                                         stream), "dfq_interleave_gate_up")
    }

    /// Per verify pass: h[rows, hidden] = silu(x . Wg^T) * (x . Wu^T) in one launch over the
    /// interleaved gate|up arrays (the MLP of DFlashDecoderLayer.swift:26 before its down
    /// projection); x is bf16 [rows, K].
    public func gateUpSiLU(x: DeviceArray, weight: DeviceArray, scales: DeviceArray,
                           biases: DeviceArray, hidden: Int, bits: Int,
                           groupSize: Int) throws -> DeviceArray {
        let inputFeatures = x.shape[x.shape.count - 1]
        let rows = x.count / inputFeatures
        var need = 0
        try check(dfq_qmm_workspace_bytes(handle, Int32(rows), Int32(2 * hidden),
                                          Int32(inputFeatures), Int32(bits), Int32(groupSize),
                                          &need), "dfq_qmm_workspace_bytes")
        let ws = workspace(need)
        let h = try DeviceBuffer(context: self, shape: [rows, hidden], dtype: .bfloat16)
        try check(dfq_qmm_silu_gate_up(handle, x.deviceAddress,
                                       weight.deviceAddress.assumingMemoryBound(to: UInt32.self),
                                       scales.deviceAddress, biases.deviceAddress, nil,
                                       h.deviceAddress, Int32(rows), Int32(hidden),
                                       Int32(inputFeatures), Int32(bits), Int32(groupSize),
                                       DFQ_BF16, ws?.0, ws?.1 ?? 0, stream),
                  "dfq_qmm_silu_gate_up")
        return h
    }
}

// MARK: - The verify round's greedy accept

/// The LM head fused with acceptedPrefix(targetLogits:proposals:)
/// (DFlashSpeculativeGenerator.swift:555-571): for the verify rows' final hidden states,
/// each row's argmax token (first index on ties, -1 for a row with no number) and the length
/// of the leading run of proposals matching them.  Only these M + 1 integers leave the
/// device; the logits are not written.
public func greedyAccept(lmHead: QuantizedLinear, hidden: DeviceArray,
                         proposals: [Int32]) throws -> (tokens: [Int32], accepted: Int) {
    let context = lmHead.context
    let h = context.handle
    let (vocab, inputFeatures) = lmHead.shape
    let rows = hidden.count / inputFeatures
    precondition(proposals.count == max(0, rows - 1), "one proposal per verify row but the last")
    guard let biases = lmHead.biases else {
        throw DFQError(status: DFQ_ERR_UNSUPPORTED, call: "greedyAccept",
                       message: "the LM head must be affine-quantised with biases")
    }
    /* the buffers of this verify width, made once per context: the workspace (in 4-byte
     * words, cleared when made; every call leaves it zero), the tokens followed by the
     * accepted count, and the proposals */
    if context.acceptBuffers[rows] == nil {
        var need = 0
        try check(dfq_qmm_argmax_accept_workspace_bytes(h, Int32(rows), Int32(vocab),
                                                        Int32(inputFeatures), Int32(lmHead.bits),
                                                        Int32(lmHead.groupSize), &need),
                  "dfq_qmm_argmax_accept_workspace_bytes")
        let wsBytes = max(1, (need + 3) / 4) * 4
        var ws: UnsafeMutableRawPointer?, out: UnsafeMutableRawPointer?
        var props: UnsafeMutableRawPointer?
        try check(dfq_malloc(h, wsBytes, &ws), "dfq_malloc")
        try check(dfq_malloc(h, (rows + 1) * 4, &out), "dfq_malloc")
        try check(dfq_malloc(h, max(1, rows - 1) * 4, &props), "dfq_malloc")
        try check(dfq_workspace_clear(h, ws, wsBytes, context.stream), "dfq_workspace_clear")
        context.acceptBuffers[rows] = (ws!, wsBytes, out!, props!)
    }
    let b = context.acceptBuffers[rows]!
    if !proposals.isEmpty {
        try proposals.withUnsafeBytes {
            try check(dfq_memcpy_h2d(h, b.props, $0.baseAddress, $0.count, context.stream),
                      "dfq_memcpy_h2d")
        }
    }
    let tokens = b.out.assumingMemoryBound(to: Int32.self)
    let proposalsOnDevice: UnsafePointer<Int32>? =
        proposals.isEmpty ? nil : UnsafePointer(b.props.assumingMemoryBound(to: Int32.self))
    try check(dfq_qmm_argmax_accept(h, hidden.deviceAddress,
                                    lmHead.weight.deviceAddress.assumingMemoryBound(to: UInt32.self),
                                    lmHead.scales.deviceAddress, biases.deviceAddress,
                                    lmHead.bias?.deviceAddress, nil, Int32(rows), Int32(vocab),
                                    Int32(inputFeatures), Int32(lmHead.bits),
                                    Int32(lmHead.groupSize), hidden.dtype.dfq, proposalsOnDevice,
                                    tokens, tokens + rows, b.ws, b.wsBytes, context.stream),
              "dfq_qmm_argmax_accept")
    var host = [Int32](repeating: 0, count: rows + 1)
    try host.withUnsafeMutableBytes {
        try check(dfq_memcpy_d2h(h, $0.baseAddress, b.out, $0.count, context.stream),
                  "dfq_memcpy_d2h")
    }
    return (Array(host[0..<rows]), Int(host[rows]))
}
