// The HIP attention path for the reference's Swift package: the attention backend seam
// (Sources/LTXAttention/AttentionBackend.swift) filled with libltx_attn.so on an MI355X.
//
// Uncompiled here: the build image has no Swift toolchain. The C target it imports
// (Sources/CLTXHip) is compiled and checked against the library's header.

import CLTXHip

/// The MI355X attention: QK-RMSNorm -> split -> split RoPE -> SDPA (-> per-head gate),
/// `DiTAttention.swift:358-381` and `:395-399`, in one asynchronous library call on device
/// buffers the caller owns. Nothing here allocates except `HIPBuffer` and `HIPWorkspace`.
public enum HIPAttention {
    /// Library failures, in the style of `DiTAttention.Failure` (`DiTAttention.swift:107-121`).
    public enum Failure: Error, CustomStringConvertible {
        case invalid(String), unsupported(String), hip(String), workspace(String)
        case noDevice(String)

        public var description: String {
            switch self {
            case let .invalid(m), let .unsupported(m), let .hip(m), let .workspace(m),
                 let .noDevice(m):
                return m
            }
        }
    }

    /// A bf16 device tensor with element strides (batch, row, head).
    public struct Tensor {
        public var data: UnsafeRawPointer
        public var batchStride: Int64, rowStride: Int64, headStride: Int64
        public init(data: UnsafeRawPointer, batchStride: Int64, rowStride: Int64,
                    headStride: Int64) {
            self.data = data
            self.batchStride = batchStride
            self.rowStride = rowStride
            self.headStride = headStride
        }
        /// The merged projection layout `[B, T, inner]` split into heads of `headDim`.
        public static func merged(_ data: UnsafeRawPointer, tokens: Int, inner: Int,
                                  headDim: Int) -> Tensor {
            Tensor(data: data, batchStride: Int64(tokens * inner), rowStride: Int64(inner),
                   headStride: Int64(headDim))
        }
    }

    /// bf16 cos / sin tables `[heads, tokens, headDim/2]` on the device (the reference's
    /// `[1, heads, tokens, headDim/2]`, broadcast over the batch).
    public struct Rotary {
        public var cos: UnsafeRawPointer, sin: UnsafeRawPointer
        public init(cos: UnsafeRawPointer, sin: UnsafeRawPointer) {
            self.cos = cos
            self.sin = sin
        }
    }

    /// Recorded beside a render like `Renderer.attentionProvenance` (`Renderer.swift:477-490`).
    public static var provenance: String { String(cString: ltx_attn_provenance()) }

    static func check(_ s: ltx_attn_status) throws {
        guard s != LTX_ATTN_OK else { return }
        let detail = String(cString: ltx_attn_last_error())
        switch s {
        case LTX_ATTN_EUNSUPPORTED: throw Failure.unsupported(detail)
        case LTX_ATTN_EHIP: throw Failure.hip(detail)
        case LTX_ATTN_EWORKSPACE: throw Failure.workspace(detail)
        default: throw Failure.invalid(detail)
        }
    }

    static func checkHIP(_ code: Int32, _ what: String) throws {
        guard code != 0 else { return }
        throw Failure.hip("\(what): \(String(cString: cltx_error_string(code)))")
    }

    /// One call's arguments, shared by `workspaceBytes` and `attend`.
    public struct Call {
        public var batch: Int32, heads: Int32, headDim: Int32
        public var queryTokens: Int32, keyTokens: Int32
        public var q: Tensor, k: Tensor, v: Tensor
        public var qNormWeight: UnsafeRawPointer?, kNormWeight: UnsafeRawPointer?
        public var rotary: Rotary?, keyRotary: Rotary?
        public var keyValidLength: [Int32]?
        public var gateLogits: Tensor?     // to_gate_logits(x): [B, Tq, heads], headStride 1
        public var out: UnsafeMutableRawPointer
        public var outStrides: (Int64, Int64, Int64)

        public init(batch: Int32, heads: Int32, headDim: Int32, queryTokens: Int32,
                    keyTokens: Int32, q: Tensor, k: Tensor, v: Tensor,
                    qNormWeight: UnsafeRawPointer?, kNormWeight: UnsafeRawPointer?,
                    rotary: Rotary?, keyRotary: Rotary?, keyValidLength: [Int32]? = nil,
                    gateLogits: Tensor? = nil, out: UnsafeMutableRawPointer,
                    outStrides: (Int64, Int64, Int64)) {
            self.batch = batch; self.heads = heads; self.headDim = headDim
            self.queryTokens = queryTokens; self.keyTokens = keyTokens
            self.q = q; self.k = k; self.v = v
            self.qNormWeight = qNormWeight; self.kNormWeight = kNormWeight
            self.rotary = rotary; self.keyRotary = keyRotary
            self.keyValidLength = keyValidLength; self.gateLogits = gateLogits
            self.out = out; self.outStrides = outStrides
        }

        func args() -> ltx_attn_args {
            var a = ltx_attn_args()
            ltx_attn_args_init(&a)
            a.B = batch; a.H = heads; a.D = headDim; a.Lq = queryTokens; a.Lk = keyTokens
            a.q = q.data; a.q_bs = q.batchStride; a.q_rs = q.rowStride; a.q_hs = q.headStride
            a.k = k.data; a.k_bs = k.batchStride; a.k_rs = k.rowStride; a.k_hs = k.headStride
            a.v = v.data; a.v_bs = v.batchStride; a.v_rs = v.rowStride; a.v_hs = v.headStride
            a.q_norm_w = qNormWeight; a.k_norm_w = kNormWeight
            a.norm_eps = 1e-6                                        // DiTAttention.swift:66
            if let r = rotary { a.q_cos = r.cos; a.q_sin = r.sin }
            if let r = keyRotary { a.k_cos = r.cos; a.k_sin = r.sin }
            a.scale = Float(1.0 / Double(headDim).squareRoot())      // DiTAttention.swift:372
            a.out = out; (a.o_bs, a.o_rs, a.o_hs) = outStrides
            if let g = gateLogits {                                   // DiTAttention.swift:395-399
                a.gate_logits = g.data; a.g_bs = g.batchStride; a.g_rs = g.rowStride; a.g_hs = 1
            }
            return a
        }

        func withArgs<R>(_ body: (inout ltx_attn_args) throws -> R) rethrows -> R {
            var a = args()
            precondition(MemoryLayout<ltx_attn_args>.size == ltx_attn_args_size(),
                         "ltx_attn_args layout differs from the library's")
            guard let lens = keyValidLength else { return try body(&a) }
            return try lens.withUnsafeBufferPointer { p in
                a.k_valid_len = p.baseAddress
                return try body(&a)
            }
        }
    }

    /// Bytes of workspace `attend` needs for this call (a pure host computation).
    public static func workspaceBytes(_ call: Call) throws -> Int {
        try call.withArgs { a in
            let n = ltx_attn_workspace_bytes(&a)
            if n == 0 { try check(ltx_attn_validate(&a)) }
            return Int(n)
        }
    }

    /// Enqueue the call on `stream` (`DiTAttention.swift:358-381`, the gate of `:395-399`
    /// when `gateLogits` is given). Inputs must stay alive until the stream passes it.
    public static func attend(_ call: Call, workspace: UnsafeMutableRawPointer?,
                              workspaceBytes: Int, stream: UnsafeMutableRawPointer?) throws {
        try call.withArgs { a in
            a.workspace = workspace
            a.workspace_bytes = workspaceBytes
            try check(ltx_attn_fwd(&a, stream))
        }
    }

    /// `linear(_:_:)` (`DiTAttention.swift:178-188`) without LoRA: y [M, N] = x [M, K] .
    /// w [N, K]^T (+ bias), bf16; with `sumsq`, the fp32 [M, ceil(N/256)] partial sums of
    /// squares of y's rows that `Call` can take in place of the norm's own statistic pass.
    /// `workspace` (at least `linearWorkspaceBytes` bytes, or nil) lets the tail tiles split.
    public static func linear(rows: Int32, outFeatures: Int32, inFeatures: Int32,
                              x: UnsafeRawPointer, xRowStride: Int64,
                              weight: UnsafeRawPointer, bias: UnsafeRawPointer?,
                              y: UnsafeMutableRawPointer, yRowStride: Int64,
                              sumsq: UnsafeMutablePointer<Float>?,
                              workspace: UnsafeMutableRawPointer? = nil, workspaceBytes: Int = 0,
                              stream: UnsafeMutableRawPointer?) throws {
        var a = ltx_linear_args()
        a.M = rows; a.N = outFeatures; a.K = inFeatures
        a.x = x; a.w = weight; a.bias = bias; a.y = y
        a.x_rs = xRowStride; a.w_rs = Int64(inFeatures); a.y_rs = yRowStride
        a.sumsq = sumsq; a.sumsq_rs = Int64(ltx_linear_sumsq_blocks(outFeatures))
        a.workspace = workspace; a.workspace_bytes = workspaceBytes
        try check(ltx_linear(&a, stream))
    }

    /// Scratch bytes that let `linear` split its tail tiles along K (0: none needed).
    public static func linearWorkspaceBytes(rows: Int32, outFeatures: Int32,
                                            inFeatures: Int32) -> Int {
        var a = ltx_linear_args()
        a.M = rows; a.N = outFeatures; a.K = inFeatures
        return ltx_linear_workspace_bytes(&a)
    }
}

/// The Gemma-4 text encoder's attention (`GemmaTextEncoder.swift:158-239`, with the mask of
/// `:288-321`) through `ltx_gemma_attn_fwd`: from the q/k/v projections to the merged output
/// before `o_proj`, fp32. Per head over D: q and k RMS-normed with their weights, v with none;
/// `rotate_half` RoPE from the layer's tables; the KV-head repeat (GQA); scale 1.0; causal,
/// sliding-window and left-padding mask, fully masked rows attending to every key.
public enum HIPGemmaAttention {
    /// One call's arguments (device pointers, element strides).
    public struct Call {
        public var batch: Int32, tokens: Int32
        public var queryHeads: Int32, keyValueHeads: Int32, headDim: Int32
        /// bf16 projections [B, T, heads * D]; `v == k` on the K-shares-V layers (V from the
        /// pre-norm K projection, `:183-188`).
        public var q: UnsafeRawPointer, k: UnsafeRawPointer, v: UnsafeRawPointer
        public var qRowStride: Int64, kRowStride: Int64, vRowStride: Int64
        public var qNormWeight: UnsafeRawPointer, kNormWeight: UnsafeRawPointer   // bf16 [D]
        public var eps: Float
        /// fp32 [T, D/2]: the first half of the layer's duplicated cos / sin rows (`:135-145`).
        public var cos: UnsafeRawPointer, sin: UnsafeRawPointer
        /// Sliding window (keys q - window < k <= q), 0 for the full layers.
        public var window: Int32
        /// Left padding per batch row (keys below are padding), or nil for none.
        public var leftPadding: [Int32]?
        /// `GemmaAttentionSpec.attentionScaling`.
        public var scale: Float
        /// fp32 [B, T, queryHeads * D].
        public var out: UnsafeMutableRawPointer

        public init(batch: Int32, tokens: Int32, queryHeads: Int32, keyValueHeads: Int32,
                    headDim: Int32, q: UnsafeRawPointer, k: UnsafeRawPointer,
                    v: UnsafeRawPointer, qRowStride: Int64, kRowStride: Int64,
                    vRowStride: Int64, qNormWeight: UnsafeRawPointer,
                    kNormWeight: UnsafeRawPointer, eps: Float, cos: UnsafeRawPointer,
                    sin: UnsafeRawPointer, window: Int32, leftPadding: [Int32]?,
                    scale: Float = 1.0, out: UnsafeMutableRawPointer) {
            self.batch = batch; self.tokens = tokens
            self.queryHeads = queryHeads; self.keyValueHeads = keyValueHeads
            self.headDim = headDim
            self.q = q; self.k = k; self.v = v
            self.qRowStride = qRowStride; self.kRowStride = kRowStride
            self.vRowStride = vRowStride
            self.qNormWeight = qNormWeight; self.kNormWeight = kNormWeight
            self.eps = eps; self.cos = cos; self.sin = sin
            self.window = window; self.leftPadding = leftPadding
            self.scale = scale; self.out = out
        }

        func withArgs<R>(_ body: (inout ltx_gemma_attn_args) throws -> R) rethrows -> R {
            var a = ltx_gemma_attn_args()
            a.B = batch; a.T = tokens; a.Hq = queryHeads; a.Hkv = keyValueHeads; a.D = headDim
            a.q = q; a.k = k; a.v = v
            a.q_rs = qRowStride; a.k_rs = kRowStride; a.v_rs = vRowStride
            a.q_bs = qRowStride * Int64(tokens); a.k_bs = kRowStride * Int64(tokens)
            a.v_bs = vRowStride * Int64(tokens)
            a.q_norm_w = qNormWeight; a.k_norm_w = kNormWeight; a.eps = eps
            a.cos = cos.assumingMemoryBound(to: Float.self)
            a.sin = sin.assumingMemoryBound(to: Float.self)
            a.window = window; a.scale = scale
            a.out = out.assumingMemoryBound(to: Float.self)
            a.o_rs = Int64(queryHeads * headDim); a.o_bs = a.o_rs * Int64(tokens)
            guard let pad = leftPadding else { return try body(&a) }
            return try pad.withUnsafeBufferPointer { p in
                a.first_valid = p.baseAddress
                return try body(&a)
            }
        }
    }

    /// Bytes of workspace `attend` needs (a pure host computation).
    public static func workspaceBytes(_ call: Call) throws -> Int {
        try call.withArgs { a in
            let n = ltx_gemma_attn_workspace_bytes(&a)
            guard n > 0 else {
                throw HIPAttention.Failure.invalid(String(cString: ltx_attn_last_error()))
            }
            return Int(n)
        }
    }

    /// Enqueue the call on `stream`. Inputs must stay alive until the stream passes it.
    public static func attend(_ call: Call, workspace: UnsafeMutableRawPointer,
                              workspaceBytes: Int, stream: UnsafeMutableRawPointer?) throws {
        try call.withArgs { a in
            a.workspace = workspace
            a.workspace_bytes = workspaceBytes
            try HIPAttention.check(ltx_gemma_attn_fwd(&a, stream))
        }
    }
}

/// Device memory owned by Swift (freed with the object).
public final class HIPBuffer {
    public let pointer: UnsafeMutableRawPointer
    public let bytes: Int

    public init(bytes: Int) throws {
        var p: UnsafeMutableRawPointer?
        try HIPAttention.checkHIP(cltx_alloc(max(bytes, 256), &p), "device allocation")
        pointer = p!
        self.bytes = bytes
    }

    deinit { _ = cltx_free(pointer) }
}

/// Page-locked host memory owned by Swift (freed with the object): copies from and to it are
/// asynchronous and need no staging copy by the runtime.
public final class HIPHostBuffer {
    public let pointer: UnsafeMutableRawPointer
    public let bytes: Int

    public init(bytes: Int) throws {
        var p: UnsafeMutableRawPointer?
        try HIPAttention.checkHIP(cltx_host_alloc(max(bytes, 256), &p), "host allocation")
        pointer = p!
        self.bytes = bytes
    }

    deinit { _ = cltx_host_free(pointer) }
}

/// Everything the `.hip` attention paths need at run time, created explicitly by the caller
/// for the device it selected (`HIPDevice.select`): one stream, a workspace, and one pair of
/// arenas -- page-locked host memory and device memory of the same size -- that hold a call's
/// operands and result at the same offsets on both sides. All three grow to the largest call
/// seen and are reused after that: a call allocates nothing once the context has seen a call
/// as large. The reference runs its model on one worker task and does not share MLX across
/// threads (`DistilledRenderer.swift:441-446`); a context follows the same rule, one per
/// worker, and calls on it run one at a time.
public final class HIPAttentionContext {
    public let ordinal: Int32
    public let stream: UnsafeMutableRawPointer
    private var workspaceBuffer: HIPBuffer?
    private var deviceArena: HIPBuffer?
    private var hostArena: HIPHostBuffer?

    /// Offsets of one call's operands in the arenas, each 256-byte aligned.
    public struct Layout {
        public private(set) var bytes = 0
        public init() {}
        /// Reserve `count` bytes; returns their offset.
        public mutating func place(_ count: Int) -> Int {
            let offset = bytes
            bytes = (offset + count + 255) / 256 * 256
            return offset
        }
    }

    public init(ordinal: Int32) throws {
        try HIPAttention.checkHIP(cltx_set_device(ordinal), "select device \(ordinal)")
        var s: UnsafeMutableRawPointer?
        try HIPAttention.checkHIP(cltx_stream_create(&s), "stream")
        self.ordinal = ordinal
        self.stream = s!
    }

    deinit {
        _ = cltx_stream_synchronize(stream)
        _ = cltx_stream_destroy(stream)
    }

    /// A workspace of at least `bytes` (the previous one when it is large enough).
    public func workspace(bytes: Int) throws -> HIPBuffer? {
        if bytes == 0 { return nil }
        if let w = workspaceBuffer, w.bytes >= bytes { return w }
        try synchronize()                  // the old buffer may still be in use on the stream
        workspaceBuffer = try HIPBuffer(bytes: bytes)
        return workspaceBuffer
    }

    /// The two arenas, at least `bytes` each: the host side to fill before `upload`, the
    /// device side the call reads and writes. Grown (after the stream has drained) only when
    /// a call needs more than any before it.
    public func arenas(bytes: Int) throws
        -> (host: UnsafeMutableRawPointer, device: UnsafeMutableRawPointer) {
        if let h = hostArena, let d = deviceArena, h.bytes >= bytes, d.bytes >= bytes {
            return (h.pointer, d.pointer)
        }
        try synchronize()
        let size = max(bytes, (hostArena?.bytes ?? 0) * 5 / 4)
        hostArena = nil
        deviceArena = nil
        hostArena = try HIPHostBuffer(bytes: size)
        deviceArena = try HIPBuffer(bytes: size)
        return (hostArena!.pointer, deviceArena!.pointer)
    }

    /// The host arena's first `bytes` to the device arena, asynchronously on the stream; the
    /// host side stays untouched until `download` has synchronised.
    public func upload(bytes: Int) throws {
        guard let h = hostArena, let d = deviceArena, bytes <= h.bytes else {
            throw HIPAttention.Failure.invalid("upload of \(bytes) bytes past the arenas")
        }
        try HIPAttention.checkHIP(cltx_upload(d.pointer, h.pointer, bytes, stream), "upload")
    }

    /// Bytes [offset, offset + bytes) of the device arena back to the same range of the host
    /// arena, then wait for the stream: the result is readable at `host + offset`.
    public func download(offset: Int, bytes: Int) throws {
        guard let h = hostArena, let d = deviceArena, offset + bytes <= h.bytes else {
            throw HIPAttention.Failure.invalid("download of \(bytes) bytes past the arenas")
        }
        try HIPAttention.checkHIP(cltx_download(h.pointer + offset, d.pointer + offset, bytes,
                                                stream), "download")
        try synchronize()
    }

    public func synchronize() throws {
        try HIPAttention.checkHIP(cltx_stream_synchronize(stream), "stream synchronize")
    }
}
