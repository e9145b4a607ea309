// The `.hip` case of `DiTAttention.AttentionPath`: the arithmetic of DiTAttention.swift:358-381
// (q_norm / k_norm over the inner dim, the head split, split RoPE, SDPA with 1/sqrt(D)) on the
// selected MI355X through libltx_attn.so, returning the same `[B, heads, T, dimHead]` tensor
// the MLX paths produce, so the gate, merge and `to_out` that follow (:385-404) are unchanged.
//
// MLX arrays live in host memory where MLX has no GPU backend, so each call copies its
// operands into the context's page-locked arena, moves the arena to the device in one
// asynchronous copy, runs the attention and copies the result back; a port that keeps its
// activations in HIP memory calls `HIPAttention.attend` on device tensors directly and moves
// nothing. The arenas and the workspace are the context's, reused from call to call.
//
// Uncompiled here: the build image has no Swift toolchain.

import Foundation
import LTXAttention
import LTXHardware
import MLX

enum HIPDiTCore {
    private final class Contexts: @unchecked Sendable {
        let lock = NSLock()
        var byOrdinal: [Int32: HIPAttentionContext] = [:]
    }
    private static let contexts = Contexts()

    /// The context of the explicitly selected device (`HIPDevice.select`). A render that
    /// chose `.hip` without selecting a device fails here, by name, before any arithmetic.
    static func context() throws -> HIPAttentionContext {
        guard let device = HIPDevice.selected else {
            throw HIPAttention.Failure.noDevice(
                "attentionPath .hip needs a device: call HIPDevice.select(ordinal:) first")
        }
        contexts.lock.lock()
        defer { contexts.lock.unlock() }
        if let c = contexts.byOrdinal[device.ordinal] { return c }
        let c = try HIPAttentionContext(ordinal: device.ordinal)
        contexts.byOrdinal[device.ordinal] = c
        return c
    }

    /// The raw bf16 bit patterns of `a`, row-major.
    static func bits(_ a: MLXArray) -> [UInt16] {
        a.asType(.bfloat16).view(dtype: .uint16).flattened().asArray(UInt16.self)
    }

    /// Copy `a`'s bf16 bits into the host arena at `offset` (exactly `count` elements).
    static func stage(_ a: MLXArray, count: Int, into host: UnsafeMutableRawPointer,
                      at offset: Int) throws {
        let b = bits(a)
        guard b.count == count else {
            throw HIPAttention.Failure.invalid("operand of \(b.count) elements, expected \(count)")
        }
        b.withUnsafeBytes { src in
            (host + offset).copyMemory(from: src.baseAddress!, byteCount: src.count)
        }
    }

    /// Tables `[1, heads, tokens, dimHead/2]` (what `DiTForward.rotaries` builds) are the
    /// library's batch-broadcast `[heads, tokens, dimHead/2]`.
    private static func checkTable(_ t: MLXArray, heads: Int, tokens: Int, half: Int) throws {
        guard t.ndim == 4, t.dim(0) == 1, t.dim(1) == heads, t.dim(2) == tokens,
              t.dim(3) == half else {
            throw DiTAttention.Failure.shape("rotary table", got: t.shape,
                                             expected: "[1, \(heads), \(tokens), \(half)]")
        }
    }

    /// Pre-norm projections `q` `[B, Tq, inner]`, `k`, `v` `[B, Tk, inner]`, the module's
    /// norm weights `[inner]` and its rotary pair(s) -> attention output `[B, heads, Tq, D]`.
    static func attend(q: MLXArray, k: MLXArray, v: MLXArray, qNorm: MLXArray, kNorm: MLXArray,
                       heads: Int, rotary: DiTAttention.Rotary?,
                       keyRotary: DiTAttention.Rotary?) throws -> MLXArray {
        let ctx = try context()
        let B = q.dim(0), Tq = q.dim(1), inner = q.dim(2), Tk = k.dim(1)
        let dimHead = inner / heads
        let half = dimHead / 2
        if let r = rotary {
            try checkTable(r.cos, heads: heads, tokens: Tq, half: half)
            try checkTable(r.sin, heads: heads, tokens: Tq, half: half)
        }
        if let r = keyRotary {
            try checkTable(r.cos, heads: heads, tokens: Tk, half: half)
            try checkTable(r.sin, heads: heads, tokens: Tk, half: half)
        }

        // One layout for the host and the device arena: the inputs, then the output.
        var lay = HIPAttentionContext.Layout()
        let nq = B * Tq * inner, nk = B * Tk * inner
        let oq = lay.place(2 * nq), ok = lay.place(2 * nk), ov = lay.place(2 * nk)
        let owq = lay.place(2 * inner), owk = lay.place(2 * inner)
        let nqt = heads * Tq * half, nkt = heads * Tk * half
        let oqc = rotary == nil ? -1 : lay.place(2 * nqt)
        let oqs = rotary == nil ? -1 : lay.place(2 * nqt)
        let okc = keyRotary == nil ? -1 : lay.place(2 * nkt)
        let oks = keyRotary == nil ? -1 : lay.place(2 * nkt)
        let inputBytes = lay.bytes
        let oout = lay.place(2 * nq)

        let (host, device) = try ctx.arenas(bytes: lay.bytes)
        try stage(q, count: nq, into: host, at: oq)
        try stage(k, count: nk, into: host, at: ok)
        try stage(v, count: nk, into: host, at: ov)
        try stage(qNorm, count: inner, into: host, at: owq)
        try stage(kNorm, count: inner, into: host, at: owk)
        var pe: HIPAttention.Rotary?
        var kpe: HIPAttention.Rotary?
        if let r = rotary {
            try stage(r.cos, count: nqt, into: host, at: oqc)
            try stage(r.sin, count: nqt, into: host, at: oqs)
            pe = HIPAttention.Rotary(cos: device + oqc, sin: device + oqs)
        }
        if let r = keyRotary {
            try stage(r.cos, count: nkt, into: host, at: okc)
            try stage(r.sin, count: nkt, into: host, at: oks)
            kpe = HIPAttention.Rotary(cos: device + okc, sin: device + oks)
        }
        try ctx.upload(bytes: inputBytes)

        let call = HIPAttention.Call(
            batch: Int32(B), heads: Int32(heads), headDim: Int32(dimHead),
            queryTokens: Int32(Tq), keyTokens: Int32(Tk),
            q: .merged(device + oq, tokens: Tq, inner: inner, headDim: dimHead),
            k: .merged(device + ok, tokens: Tk, inner: inner, headDim: dimHead),
            v: .merged(device + ov, tokens: Tk, inner: inner, headDim: dimHead),
            qNormWeight: device + owq, kNormWeight: device + owk,
            rotary: pe, keyRotary: kpe,
            out: device + oout,
            outStrides: (Int64(Tq * inner), Int64(inner), Int64(dimHead)))
        let bytes = try HIPAttention.workspaceBytes(call)
        let ws = try ctx.workspace(bytes: bytes)
        try HIPAttention.attend(call, workspace: ws?.pointer, workspaceBytes: bytes,
                                stream: ctx.stream)
        try ctx.download(offset: oout, bytes: 2 * nq)
        let result = Array(UnsafeBufferPointer(
            start: (host + oout).assumingMemoryBound(to: UInt16.self), count: nq))
        // [B, Tq, inner] -> [B, heads, Tq, dimHead], the layout `split` gives (:346-349)
        return MLXArray(result).reshaped([B, Tq, heads, dimHead]).view(dtype: .bfloat16)
            .transposed(0, 2, 1, 3)
    }
}
