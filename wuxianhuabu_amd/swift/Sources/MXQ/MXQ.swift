// MXQ: the MLX-Swift quantized-linear operators the reference calls, over libmxq's C ABI.
//
//   quantized(_:groupSize:bits:)       mx.quantize
//                                      (`model/minimax h3/tools/quantize_h3_g64.py:132`),
//                                      quantize(model:)
//                                      (`Packages/z-image-swift/Sources/ZImage/Weights.swift:31`)
//   dequantized(_:scales:biases:...)   `model/minimax h3/H3Common.swift:382-401`
//   quantizedMatmul / quantizedMM      `model/minimax h3/H3Common.swift:358-359`,
//                                      `model/3模块/ltx2.5专属/gemma4文本-(ltx专属).swift:306-312`
//   QuantizedLinear                    `model/3模块/ltx2.5专属/ltx主干-(ltx专属).swift:177-188`
//   MfLinear.load / forward            `model/minimax h3/H3Common.swift:283-377`
//   SafetensorsFile                    `model/minimax h3/H3Common.swift:181-260`
//
// Arrays live in device memory (DeviceArray). Every operation is enqueued on a Stream and
// returns without waiting; a DeviceArray's memory is freed only after the stream it was
// last used on has finished, the rule the reference keeps around buffer release
// (`model/minimax h3/H3Pipeline.swift:212-228`, Stream.gpu.synchronize() first). An array
// used on several streams must be synchronized by its user on all but the last one.
import CMXQ

public struct MXQError: Error, CustomStringConvertible {
    public let status: Int32
    public let message: String
    public var description: String {
        "\(String(cString: mxq_status_string(status))): \(message)"
    }
}

@inline(__always)
func check(_ rc: Int32) throws {
    if rc != MXQ_OK {
        throw MXQError(status: rc, message: String(cString: mxq_last_error()))
    }
}

/// A HIP stream of default priority, owned by the bridge.
public final class Stream {
    public let raw: mxq_stream?

    public init() throws {
        var s: mxq_stream? = nil
        try check(mxq_stream_create(&s))
        raw = s
    }

    public func synchronize() throws { try check(mxq_stream_synchronize(raw)) }

    deinit {
        _ = mxq_stream_synchronize(raw)
        _ = mxq_stream_destroy(raw)
    }

    /// The stream operations use when none is given.
    public static let gpu: Stream = try! Stream()
}

public enum DType {
    case uint32, bfloat16, float32, uint8

    public var size: Int {
        switch self {
        case .uint32, .float32: return 4
        case .bfloat16: return 2
        case .uint8: return 1
        }
    }

    var code: Int32 { self == .float32 ? MXQ_FLOAT32 : MXQ_BFLOAT16 }
}

/// A row-major tensor in device memory.
public final class DeviceArray {
    public let ptr: UnsafeMutableRawPointer?
    public let shape: [Int]
    public let dtype: DType
    /// The stream of the last operation that read or wrote this array; deinit waits for it.
    public internal(set) var stream: Stream

    public var count: Int { shape.reduce(1, *) }
    public var nbytes: Int { count * dtype.size }

    public init(shape: [Int], dtype: DType, stream: Stream = .gpu) throws {
        self.shape = shape
        self.dtype = dtype
        self.stream = stream
        var p: UnsafeMutableRawPointer? = nil
        try check(mxq_malloc(&p, shape.reduce(1, *) * dtype.size))
        ptr = p
    }

    /// Copies `bytes` (host memory, nbytes long) into a new device array.
    public convenience init(host bytes: UnsafeRawBufferPointer, shape: [Int], dtype: DType,
                            stream: Stream = .gpu) throws {
        try self.init(shape: shape, dtype: dtype, stream: stream)
        precondition(bytes.count == nbytes, "host buffer size does not match the shape")
        try check(mxq_copy_to_device(ptr, bytes.baseAddress, nbytes, stream.raw))
    }

    /// The array's bytes, copied to host memory once all work on its stream is done.
    public func hostBytes() throws -> [UInt8] {
        var out = [UInt8](repeating: 0, count: nbytes)
        try out.withUnsafeMutableBytes { buf in
            try check(mxq_copy_to_host(buf.baseAddress, ptr, nbytes, stream.raw))
        }
        return out
    }

    func used(on s: Stream) { stream = s }

    var u32: UnsafeMutablePointer<UInt32>? { ptr?.assumingMemoryBound(to: UInt32.self) }

    deinit {
        if ptr != nil {
            _ = mxq_stream_synchronize(stream.raw)
            _ = mxq_free(ptr)
        }
    }
}

public enum QuantizationMode {
    /// mlx's affine quantizer (sign-aware, the group's larger-magnitude extreme on code 0)
    case affine
    /// scale = (max - min) / (2^bits - 1), bias = min
    case minmax

    var code: Int32 { self == .affine ? MXQ_MODE_MLX_EDGE : MXQ_MODE_MINMAX }
}

// MARK: - operators

/// Quantizes w [..., K] along its last axis. scales/biases take w's dtype.
public func quantized(_ w: DeviceArray, groupSize: Int = 64, bits: Int = 4,
                      mode: QuantizationMode = .affine, stream: Stream = .gpu) throws
    -> (wq: DeviceArray, scales: DeviceArray, biases: DeviceArray)
{
    guard let K = w.shape.last, w.shape.count >= 2, w.dtype == .float32 || w.dtype == .bfloat16
    else {
        throw MXQError(status: MXQ_ERR_INVALID, message: "[quantize] need a float [..., K] matrix")
    }
    let lead = Array(w.shape.dropLast())
    let rows = lead.reduce(1, *)
    let wq = try DeviceArray(shape: lead + [K * bits / 32], dtype: .uint32, stream: stream)
    let s = try DeviceArray(shape: lead + [K / max(groupSize, 1)], dtype: w.dtype,
                            stream: stream)
    let b = try DeviceArray(shape: s.shape, dtype: w.dtype, stream: stream)
    try check(mxq_quantize(w.ptr, w.dtype.code, Int64(rows), Int64(K), Int32(groupSize),
                           Int32(bits), mode.code, wq.u32, s.ptr, b.ptr, w.dtype.code,
                           stream.raw))
    for a in [w, wq, s, b] { a.used(on: stream) }
    return (wq, s, b)
}

/// w = q * scale + bias, [..., K] in scales' dtype.
public func dequantized(_ wq: DeviceArray, scales: DeviceArray, biases: DeviceArray,
                        groupSize: Int = 64, bits: Int = 4, stream: Stream = .gpu) throws
    -> DeviceArray
{
    guard let wcols = wq.shape.last else {
        throw MXQError(status: MXQ_ERR_INVALID, message: "[dequantize] empty shape")
    }
    let K = wcols * 32 / bits
    let lead = Array(wq.shape.dropLast())
    let out = try DeviceArray(shape: lead + [K], dtype: scales.dtype, stream: stream)
    try check(mxq_dequantize(wq.u32, scales.ptr, biases.ptr, scales.dtype.code,
                             Int64(lead.reduce(1, *)), Int64(K), Int32(groupSize), Int32(bits),
                             out.ptr, scales.dtype.code, stream.raw))
    for a in [wq, scales, biases, out] { a.used(on: stream) }
    return out
}

/// y [..., N] = x [..., K] · dequantized(w)ᵀ (+ bias), bf16 in and out, fp32 accumulation.
public func quantizedMatmul(_ x: DeviceArray, _ w: DeviceArray, scales: DeviceArray,
                            biases: DeviceArray, transpose: Bool = true, groupSize: Int = 64,
                            bits: Int = 4, bias: DeviceArray? = nil, stream: Stream = .gpu)
    throws -> DeviceArray
{
    guard let K = x.shape.last, w.shape.count == 2 else {
        throw MXQError(status: MXQ_ERR_INVALID, message: "[quantized_matmul] bad shapes")
    }
    let N = w.shape[0]
    let M = x.count / max(K, 1)
    let y = try DeviceArray(shape: Array(x.shape.dropLast()) + [N], dtype: .bfloat16,
                            stream: stream)
    try check(mxq_quantized_matmul(x.ptr, Int64(M), Int64(K), w.u32, scales.ptr, biases.ptr,
                                   Int64(N), transpose ? 1 : 0, Int32(groupSize), Int32(bits),
                                   bias?.ptr, y.ptr, stream.raw))
    for a in [x, w, scales, biases, y] { a.used(on: stream) }
    bias?.used(on: stream)
    return y
}

/// The spelling H3Common uses.
public func quantizedMM(_ x: DeviceArray, _ w: DeviceArray, scales: DeviceArray,
                        biases: DeviceArray, transpose: Bool = true, groupSize: Int = 64,
                        bits: Int = 4, stream: Stream = .gpu) throws -> DeviceArray
{
    try quantizedMatmul(x, w, scales: scales, biases: biases, transpose: transpose,
                        groupSize: groupSize, bits: bits, stream: stream)
}

// MARK: - the tiled copy

/// The same bits as an MLX triple, reordered once for the MFMA and GEMV kernels
/// (mxq_tile); requires K % 64 == 0 and bf16 scales/biases. Results are bit-identical
/// to the MLX-layout kernels.
public final class TiledWeight {
    public let data: DeviceArray
    public let N: Int, K: Int, groupSize: Int, bits: Int

    public static func supported(K: Int, groupSize: Int, bits: Int, scales: DType) -> Bool {
        scales == .bfloat16 && K > 0 && mxq_tiled_bytes(1, Int64(K), Int32(groupSize),
                                                        Int32(bits)) > 0
    }

    public init(wq: DeviceArray, scales: DeviceArray, biases: DeviceArray, groupSize: Int,
                bits: Int, stream: Stream = .gpu) throws
    {
        N = wq.shape[0]
        K = wq.shape[1] * 32 / bits
        self.groupSize = groupSize
        self.bits = bits
        let bytes = mxq_tiled_bytes(Int64(N), Int64(K), Int32(groupSize), Int32(bits))
        if bytes < 0 { try check(Int32(bytes)) }
        data = try DeviceArray(shape: [Int(bytes)], dtype: .uint8, stream: stream)
        try check(mxq_tile(wq.u32, scales.ptr, biases.ptr, Int64(N), Int64(K), Int32(groupSize),
                           Int32(bits), data.ptr, stream.raw))
        for a in [wq, scales, biases, data] { a.used(on: stream) }
    }

    /// The MLX triple these bits came from (mxq_untile), as new arrays.
    public func untiled(stream: Stream = .gpu) throws
        -> (wq: DeviceArray, scales: DeviceArray, biases: DeviceArray)
    {
        let wq = try DeviceArray(shape: [N, K * bits / 32], dtype: .uint32, stream: stream)
        let s = try DeviceArray(shape: [N, K / groupSize], dtype: .bfloat16, stream: stream)
        let b = try DeviceArray(shape: [N, K / groupSize], dtype: .bfloat16, stream: stream)
        try check(mxq_untile(data.ptr, Int64(N), Int64(K), Int32(groupSize), Int32(bits),
                             wq.u32, s.ptr, b.ptr, stream.raw))
        data.used(on: stream)
        return (wq, s, b)
    }

    public func matmul(_ x: DeviceArray, bias: DeviceArray?, stream: Stream = .gpu) throws
        -> DeviceArray
    {
        let M = x.count / K
        let y = try DeviceArray(shape: Array(x.shape.dropLast()) + [N], dtype: .bfloat16,
                                stream: stream)
        try check(mxq_quantized_matmul_tiled(x.ptr, Int64(M), Int64(K), data.ptr, Int64(N),
                                             Int32(groupSize), Int32(bits), bias?.ptr, y.ptr,
                                             stream.raw))
        for a in [x, data, y] { a.used(on: stream) }
        bias?.used(on: stream)
        return y
    }
}

/// One resident copy of a quantized weight: the MLX triple, or, once tiled, only the
/// tiled copy (the triple is rebuilt from it when read).
final class ResidentWeight {
    private var triple: (DeviceArray, DeviceArray, DeviceArray)?
    private(set) var tiled: TiledWeight?
    let groupSize: Int, bits: Int

    init(_ wq: DeviceArray, _ s: DeviceArray, _ b: DeviceArray, groupSize: Int, bits: Int,
         tile: Bool, stream: Stream) throws
    {
        self.groupSize = groupSize
        self.bits = bits
        let K = wq.shape[1] * 32 / bits
        if tile && TiledWeight.supported(K: K, groupSize: groupSize, bits: bits, scales: s.dtype) {
            // built at load; the triple is released once the tiling has run (DeviceArray
            // deinit waits for the stream)
            tiled = try TiledWeight(wq: wq, scales: s, biases: b, groupSize: groupSize,
                                    bits: bits, stream: stream)
        } else {
            triple = (wq, s, b)
        }
    }

    func parts(stream: Stream) throws -> (DeviceArray, DeviceArray, DeviceArray) {
        if let t = triple { return t }
        let u = try tiled!.untiled(stream: stream)
        return (u.wq, u.scales, u.biases)
    }
}

// MARK: - layers

/// MLXNN's QuantizedLinear as the LTX backbone uses it: weight / scales / biases (+ bias),
/// callAsFunction(x) = quantizedMatmul(x, weight, ..., transpose: true) + bias.
public final class QuantizedLinear {
    public let inputDims: Int, outputDims: Int, groupSize: Int, bits: Int
    public var bias: DeviceArray?
    let resident: ResidentWeight
    let stream: Stream

    public init(weight: DeviceArray, scales: DeviceArray, biases: DeviceArray,
                bias: DeviceArray? = nil, groupSize: Int = 64, bits: Int = 4,
                tiled: Bool = true, stream: Stream = .gpu) throws
    {
        outputDims = weight.shape[0]
        inputDims = weight.shape[1] * 32 / bits
        self.groupSize = groupSize
        self.bits = bits
        self.bias = bias
        self.stream = stream
        resident = try ResidentWeight(weight, scales, biases, groupSize: groupSize, bits: bits,
                                      tile: tiled, stream: stream)
    }

    public var weight: DeviceArray { get throws { try resident.parts(stream: stream).0 } }
    public var scales: DeviceArray { get throws { try resident.parts(stream: stream).1 } }
    public var biases: DeviceArray { get throws { try resident.parts(stream: stream).2 } }

    public func callAsFunction(_ x: DeviceArray) throws -> DeviceArray {
        if let t = resident.tiled, x.dtype == .bfloat16, x.shape.last == t.K {
            return try t.matmul(x, bias: bias, stream: stream)
        }
        let (w, s, b) = try resident.parts(stream: stream)
        return try quantizedMatmul(x, w, scales: s, biases: b, transpose: true,
                                   groupSize: groupSize, bits: bits, bias: bias, stream: stream)
    }
}

/// safetensors read straight into device memory (mxq_st_*), as H3Weights reads them.
public final class SafetensorsFile {
    let handle: OpaquePointer

    public init(path: String) throws {
        var h: OpaquePointer? = nil
        try check(mxq_st_open(path, &h))
        handle = h!
    }

    deinit { mxq_st_close(handle) }

    public var keys: [String] {
        (0..<Int(mxq_st_count(handle))).map { String(cString: mxq_st_key(handle, Int64($0))) }
    }

    public func get(_ key: String, stream: Stream = .gpu) throws -> DeviceArray? {
        var dt = [CChar](repeating: 0, count: 16)
        var ndim: Int32 = 0
        var shape = [Int64](repeating: 0, count: Int(MXQ_ST_MAX_DIMS))
        var nbytes: Int64 = 0
        guard mxq_st_info(handle, key, &dt, &ndim, &shape, &nbytes) == MXQ_OK else { return nil }
        let name = String(cString: dt)
        let dtype: DType = name == "U32" ? .uint32 : name == "BF16" ? .bfloat16
            : name == "F32" ? .float32 : .uint8
        let dims = shape.prefix(Int(ndim)).map { Int($0) }
        let a = try DeviceArray(shape: dtype == .uint8 ? [Int(nbytes)] : dims, dtype: dtype,
                                stream: stream)
        try check(mxq_st_read(handle, key, a.ptr, stream.raw))
        return a
    }

    /// (weight, scales, biases) under either key spelling
    /// (`model/minimax h3/H3Common.swift:249-258`).
    public func getQuantized(_ prefix: String, stream: Stream = .gpu) throws
        -> (weight: DeviceArray, scales: DeviceArray, biases: DeviceArray)?
    {
        guard let w = try get(prefix + ".weight", stream: stream) else { return nil }
        for (sk, bk) in [(".scales", ".biases"), (".weight.scales", ".weight.biases")] {
            if let s = try get(prefix + sk, stream: stream),
               let b = try get(prefix + bk, stream: stream) {
                return (w, s, b)
            }
        }
        return nil
    }
}

/// The reference's MfLinear for quantized layers: bits = 32·wCols/in, groupSize = in/sCols;
/// forward casts nothing (x is bf16) and fuses the bias into the kernel's epilogue.
public final class MfLinear {
    public let inDim: Int
    public private(set) var outDim: Int = 0
    public private(set) var bits: Int = 0
    public private(set) var groupSize: Int = 0
    public var bias: DeviceArray?
    var resident: ResidentWeight?
    let stream: Stream

    init(inDim: Int, stream: Stream) {
        self.inDim = inDim
        self.stream = stream
    }

    public static func load(_ file: SafetensorsFile, prefix: String, inFeatures: Int,
                            stream: Stream = .gpu) throws -> MfLinear
    {
        let lin = MfLinear(inDim: inFeatures, stream: stream)
        guard let q = try file.getQuantized(prefix, stream: stream) else {
            throw MXQError(status: MXQ_ERR_INVALID, message: "missing weight: \(prefix).weight")
        }
        guard q.weight.shape.count == 2, q.scales.shape.count == 2 else {
            throw MXQError(status: MXQ_ERR_INVALID, message: "bad file: quantized weight rank")
        }
        lin.outDim = q.weight.shape[0]
        lin.bits = 32 * q.weight.shape[1] / inFeatures
        lin.groupSize = inFeatures / q.scales.shape[1]
        lin.bias = try file.get(prefix + ".bias", stream: stream)
        lin.resident = try ResidentWeight(q.weight, q.scales, q.biases, groupSize: lin.groupSize,
                                          bits: lin.bits, tile: true, stream: stream)
        return lin
    }

    public func forward(_ x: DeviceArray) throws -> DeviceArray {
        guard let r = resident else {
            throw MXQError(status: MXQ_ERR_INVALID, message: "MfLinear is not loaded")
        }
        if let t = r.tiled, x.shape.last == t.K {
            return try t.matmul(x, bias: bias, stream: stream)
        }
        let (w, s, b) = try r.parts(stream: stream)
        return try quantizedMatmul(x, w, scales: s, biases: b, transpose: true,
                                   groupSize: groupSize, bits: bits, bias: bias, stream: stream)
    }

    /// The dense weight [out, in] (`model/minimax h3/H3Common.swift:382-401`).
    public func dequantizedWeight() throws -> DeviceArray {
        guard let r = resident else {
            throw MXQError(status: MXQ_ERR_INVALID, message: "MfLinear is not loaded")
        }
        let (w, s, b) = try r.parts(stream: stream)
        return try dequantized(w, scales: s, biases: b, groupSize: groupSize, bits: bits,
                               stream: stream)
    }
}
